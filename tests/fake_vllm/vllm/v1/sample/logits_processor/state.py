"""TEST-ONLY: LogitsProcessors container."""


class LogitsProcessors:
    def __init__(self, argmax_invariant=None, non_argmax_invariant=None):
        self.argmax_invariant = list(argmax_invariant or [])
        self.non_argmax_invariant = list(non_argmax_invariant or [])

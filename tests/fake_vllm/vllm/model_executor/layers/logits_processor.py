"""TEST-ONLY: upstream LogitsProcessor with its unquantized _get_logits."""
import torch


class LogitsProcessor(torch.nn.Module):
    def __init__(self, vocab_size, org_vocab_size=None, scale=1.0, logits_as_input=False, soft_cap=None):
        super().__init__()
        self.scale = scale
        self.vocab_size = vocab_size
        self.logits_as_input = logits_as_input
        self.org_vocab_size = org_vocab_size or vocab_size
        self.soft_cap = soft_cap
        self.use_all_gather = False

    def _get_logits(self, hidden_states, lm_head, embedding_bias, skip_gather=False):
        logits = torch.nn.functional.linear(hidden_states, lm_head.weight.data)
        if embedding_bias is not None:
            logits = logits + embedding_bias
        return logits[..., : self.org_vocab_size]

"""TEST-ONLY: upstream Sampler (greedy / exponential-race random sampling, top-k/top-p)."""
import torch

_SAMPLING_EPS = 1e-5


class Sampler(torch.nn.Module):
    def __init__(self, logprobs_mode="raw_logprobs"):
        super().__init__()
        self.logprobs_mode = logprobs_mode

    @staticmethod
    def apply_temperature(logits, temp, all_random):
        if not all_random:
            temp = torch.where(temp < _SAMPLING_EPS, 1.0, temp)
        return logits.div_(temp.unsqueeze(dim=1))

    @staticmethod
    def greedy_sample(logits):
        return logits.argmax(dim=-1).view(-1)

    def compute_logprobs(self, logits):
        return logits.log_softmax(dim=-1, dtype=torch.float32)

    def gather_logprobs(self, logprobs, num_logprobs, token_ids):
        return torch.topk(logprobs, num_logprobs, dim=-1)

    def sample(self, logits, sampling_metadata, logprobs_mode_override=None):
        sm = sampling_metadata
        mode = logprobs_mode_override or self.logprobs_mode
        processed = None
        greedy = None if sm.all_random else self.greedy_sample(logits)
        if sm.all_greedy:
            if mode == "processed_logits":
                processed = logits
            elif mode == "processed_logprobs":
                processed = self.compute_logprobs(logits)
            return greedy, processed
        logits = self.apply_temperature(logits.clone(), sm.temperature, sm.all_random)
        if sm.top_k is not None:
            k = int(sm.top_k.max().item())
            kth = torch.topk(logits, k, dim=-1).values.gather(-1, (sm.top_k.long() - 1).clamp(min=0).unsqueeze(-1))
            logits = logits.masked_fill(logits < kth, float("-inf"))
        if sm.top_p is not None:
            srt, idx = logits.sort(dim=-1, descending=False)
            cum = srt.softmax(dim=-1).cumsum(dim=-1)
            mask = cum <= 1 - sm.top_p.unsqueeze(1)
            mask[:, -1] = False
            srt = srt.masked_fill(mask, float("-inf"))
            logits = torch.empty_like(logits).scatter_(-1, idx, srt)
        if mode == "processed_logits":
            processed = logits
        elif mode == "processed_logprobs":
            processed = self.compute_logprobs(logits)
        probs = logits.softmax(dim=-1, dtype=torch.float32)
        q = torch.empty_like(probs).exponential_()
        for i, g in sm.generators.items():
            q[i].exponential_(generator=g)
        random = probs.div_(q).argmax(dim=-1).view(-1)
        if greedy is None:
            return random, processed
        return torch.where(sm.temperature < _SAMPLING_EPS, greedy, random), processed

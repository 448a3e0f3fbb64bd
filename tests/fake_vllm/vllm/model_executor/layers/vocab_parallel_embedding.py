"""TEST-ONLY: VocabParallelEmbedding holder of the lm_head weight."""
import torch


class VocabParallelEmbedding(torch.nn.Module):
    def __init__(self, weight: torch.Tensor):
        super().__init__()
        self.weight = torch.nn.Parameter(weight, requires_grad=False)

"""TEST-ONLY: SamplingMetadata with the fields the fused sampler reads."""
from dataclasses import dataclass, field
from typing import Any, Optional

import torch


@dataclass
class SamplingMetadata:
    temperature: Optional[torch.Tensor]
    all_greedy: bool
    all_random: bool
    top_p: Optional[torch.Tensor]
    top_k: Optional[torch.Tensor]
    generators: dict
    max_num_logprobs: Optional[int]
    no_penalties: bool
    prompt_token_ids: Optional[torch.Tensor]
    frequency_penalties: torch.Tensor
    presence_penalties: torch.Tensor
    repetition_penalties: torch.Tensor
    output_token_ids: list
    allowed_token_ids_mask: Optional[torch.Tensor]
    bad_words_token_ids: dict
    logitsprocs: Any
    logprob_token_ids: Any = None
    spec_token_ids: Any = None
    thinking_budget_state_holder: Any = None

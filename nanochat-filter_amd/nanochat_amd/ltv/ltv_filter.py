"""``LtvInitValues``: optional per-call initial filter states
(reference ``nanochat/ltv/ltv_filter.py:36-39``)."""

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class LtvInitValues:
    q: Optional[torch.Tensor] = None
    k: Optional[torch.Tensor] = None
    v: Optional[torch.Tensor] = None

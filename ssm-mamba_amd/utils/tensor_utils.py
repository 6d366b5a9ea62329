"""None-safe contiguity helper (same contract as the reference's
``utils/tensor_utils.py:3-6``)."""
from __future__ import annotations

from typing import Optional

import torch


def ensure_contiguous(x: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if x is None or x.is_contiguous():
        return x
    return x.contiguous()

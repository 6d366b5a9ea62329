"""MI355X (gfx950) selective-scan hot path for Mamba.

Drop-in operator API: ``ssm_mamba_amd.ops.SelectiveScanFn`` /
``SelectiveUpdateFn`` (the reference's classes) and the functional
``selective_scan_fn`` / ``selective_state_update``.  All compute runs in the
hand-written HIP library ``_lib/libssm_mamba_hip.so`` (C ABI in
``include/ssm_mamba.h``); there is no CPU or PyTorch fallback.
"""
from .ops import SelectiveScanFn, SelectiveUpdateFn, selective_scan_fn, selective_state_update

__all__ = ["SelectiveScanFn", "SelectiveUpdateFn", "selective_scan_fn", "selective_state_update"]
__version__ = "0.1.0"

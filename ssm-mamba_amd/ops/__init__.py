"""Operator API (mirrors the reference's ``ops/__init__.py:1-2``)."""
from .selective_scan_interface import SelectiveScanFn, selective_scan_fn
from .selective_update_interface import SelectiveUpdateFn, selective_state_update

__all__ = ["SelectiveScanFn", "SelectiveUpdateFn", "selective_scan_fn", "selective_state_update"]

"""Batched isotonic regression for PyTorch tensors on AMD MI355X: a drop-in for
``torchisotonic.isotonic`` (reference src/torchisotonic/__init__.py:3-6) backed by hand-written
HIP kernels for gfx950."""

from torchisotonic_amd._api import isotonic
from torchisotonic_amd.calibration import IsotonicCalibrator, calibration_fit, calibration_predict
from torchisotonic_amd.ragged import isotonic_ragged
from torchisotonic_amd.soft_rank import soft_rank

__all__ = ["isotonic", "isotonic_ragged", "soft_rank", "IsotonicCalibrator", "calibration_fit", "calibration_predict"]
__version__ = "0.1.0"
# The torchisotonic release whose API and semantics this package reproduces.
REFERENCE_VERSION = "0.2.1"

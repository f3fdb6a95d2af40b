"""trainscale_amd — MI355X (gfx950) fused kernel layer for TrainScale-style training.

Hot-path ops with TrainScale's signatures, backed by hand-written HIP kernels
in ``libtrainscale_amd.so`` (C ABI: ``include/trainscale_amd.h``):

* RMSNorm forward/backward (``kernels.fast_rms_layernorm`` and friends)
* RoPE forward/backward incl. packed ``position_ids`` (``kernels.apply_rope*``)
* vocabulary cross-entropy forward/backward (``kernels.fast_cross_entropy_loss``,
  ``loss.ChunkedCrossEntropyLoss``, ``loss.FusedCrossEntropyLoss``, ``loss.CrossEntropyLoss``)
"""
from . import _lib

__version__ = "0.1.0"


def library_path() -> str:
    return str(_lib.LIB_PATH)


def load_library():
    """Loads the native library now (raises if it is missing)."""
    return _lib.load()

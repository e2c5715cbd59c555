"""Loader for the MI355X extension (counterpart of src/murmurative/_cuda_kernels.py).

Importing ``murmurative_attention_ops`` (built in-tree next to this file by
``murmurative-attention_amd/build.py``) runs its static registrars, which
define ``torch.ops.murmurative_attention``.  There is no fallback: without a
GPU or without the built library every HIP entry point raises.
"""

import os

_loaded = False
HERE = os.path.dirname(os.path.abspath(__file__))
EXT_PATH = os.path.join(HERE, "murmurative_attention_ops.so")
LIB_PATH = os.path.join(HERE, "libmurmurative_hip.so")


def ensure_compiled() -> bool:
    """Load the HIP extension; RuntimeError when no GPU or no build is present."""
    global _loaded
    if _loaded:
        return True
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError(
            "murmurative HIP kernels need a ROCm GPU (MI355X / gfx950), but none is visible. "
            "Pass use_reference=True for the eager PyTorch path.")
    try:
        from . import murmurative_attention_ops  # noqa: F401  (registers the ops)
    except ImportError as exc:
        raise RuntimeError(
            "murmurative HIP extension is not built or does not load: run "
            "`python murmurative-attention_amd/build.py` (hipcc --offload-arch=gfx950).") from exc
    try:
        ns = torch.ops.murmurative_attention
        _ = ns.slot_murmurate_fwd
    except (AttributeError, RuntimeError) as exc:
        raise RuntimeError(
            "murmurative extension loaded but torch.ops.murmurative_attention is incomplete; "
            "rebuild it.") from exc
    _loaded = True
    return True

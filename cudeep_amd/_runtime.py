"""One HIP runtime per process.

PyTorch-ROCm wheels carry their own libamdhip64.so (torch/lib, found through
torch's $ORIGIN rpath), with the same soname, libamdhip64.so.7, as the ROCm
installation's copy that this package's libraries are linked against.  If
this package loads first, the dynamic loader maps /opt/rocm's runtime; a
later ``import torch`` then maps torch's copy as a second runtime (it is
found by path, not by soname), and whichever initialises second sees no GPU
("no ROCm-capable device is detected").  When torch is importable, its
runtime is therefore loaded first, globally, so this package's libraries
bind to that same object and torch, imported later or earlier, reuses it.
Without torch the ROCm installation's runtime is used as linked.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os


def share_torch_hip_runtime():
    """Preload torch's bundled HIP runtime if there is one; returns its path
    (or None).  Does not import torch."""
    try:
        spec = importlib.util.find_spec("torch")
    except (ImportError, ValueError):
        return None
    if spec is None or not spec.origin:
        return None
    path = os.path.join(os.path.dirname(spec.origin), "lib", "libamdhip64.so")
    if not os.path.exists(path):
        return None
    ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
    return path

"""Helpers shared by the GPU parity tests (host-side only)."""
import sys

import numpy as np
import pytest

try:
    import torch
except Exception:  # pragma: no cover
    torch = None


def require_gpu():
    if torch is None or not torch.cuda.is_available():
        pytest.skip("needs an MI355X GPU")


def say(*parts):
    """Names the case on stdout (flushed) before a GPU step."""
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def uniform(rng, shape, lo=-1.0, hi=1.0):
    return rng.uniform(lo, hi, shape).astype(np.float32)


def normal(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32)


# One fp32 unit roundoff: an additive floor on error gates for problems so
# small (K < 64) that the reference's own error is a handful of roundings.
F32_FLOOR = 2.0 ** -24

"""Shared helpers for the GPU parity tests (they call libpxs.so through pxs.py)."""

import numpy as np
import torch

FP32_TOL = 1e-5   # max|g - r| / max|r|
BF16_TOL = 1e-2   # relative L2


def dev():
    return torch.device("cuda:0")


def t32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev())


def ti32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev())


def ti64(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int64)).to(dev())


def tbf(a):
    """float32 numpy (already bf16-representable or not) -> bf16 device tensor (RNE)."""
    return t32(a).to(torch.bfloat16)


def host(t):
    return t.detach().float().cpu().numpy()


def max_rel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(got - ref))) / denom


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def assert_fp32(got, ref, tol=FP32_TOL, what=""):
    e = max_rel(got, ref)
    assert e <= tol, f"{what}: max rel error {e:.3e} > {tol}"


def assert_bf16(got, ref, tol=BF16_TOL, what=""):
    e = rel_l2(got, ref)
    assert e <= tol, f"{what}: rel L2 error {e:.3e} > {tol}"

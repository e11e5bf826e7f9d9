"""Helpers of the GPU parity tests: seeded inputs in f16 / bf16 (as torch tensors and as the bit patterns the
oracle reads), and the tolerance of the attention path.

Tolerance (fp16 / bf16 outputs and fp32 outputs alike): every element within |err| <= 2e-3 + 1e-2 |ref|, LSE within
1e-3 absolute (the same infinity where a row is fully masked). The reference's own figure, the worst row's
relative L2 error (tests/sparse_attn_test.cpp:174-181, threshold 5e-3), is checked beside it.
"""
import numpy as np
import torch

import oracle as O

ATOL, RTOL, LSE_TOL, ROW_L2 = 2e-3, 1e-2, 1e-3, 5e-3
TORCH = {O.F16: torch.float16, O.BF16: torch.bfloat16}


def bits(x, dtype):
    return O.to_f16_bits(x) if dtype == O.F16 else O.to_bf16_bits(x)


def randn_bits(rng, shape, dtype, scale=1.0):
    return bits(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale), dtype)


def to_dev(b, dtype):
    """uint16 bit patterns -> a torch tensor of the element type on cuda:0."""
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(TORCH[dtype]).to("cuda")


def to_host(t):
    return t.float().cpu().numpy().astype(np.float64)


def assert_attn_close(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    assert np.all(np.isfinite(got)), f"{what}: {np.sum(~np.isfinite(got))} non-finite outputs"
    err = np.abs(got - want)
    bad = err > ATOL + RTOL * np.abs(want)
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} elements out of tolerance, max abs err "
                           f"{err.max():.3e} at {np.unravel_index(np.argmax(err), err.shape)}")


def assert_rows_l2(got, want, what, dim):
    got = np.asarray(got, np.float64).reshape(-1, dim)
    want = np.asarray(want, np.float64).reshape(-1, dim)
    nrm = np.maximum((want ** 2).sum(1), 1e-30)
    worst = float(np.sqrt(((got - want) ** 2).sum(1) / nrm).max())
    nz = (want ** 2).sum(1) > 0
    worst = float(np.sqrt(((got - want) ** 2).sum(1)[nz] / nrm[nz]).max()) if nz.any() else 0.0
    assert worst < ROW_L2, f"{what}: worst row relative L2 error {worst:.2e}"


def assert_lse_close(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    inf_w, inf_g = np.isinf(want), np.isinf(got)
    assert np.array_equal(inf_w, inf_g) and np.all(np.sign(got[inf_g]) == np.sign(want[inf_w])), \
        f"{what}: fully masked rows differ"
    err = np.abs(got[~inf_w] - want[~inf_w])
    assert err.size == 0 or err.max() <= LSE_TOL, f"{what}: LSE max abs err {err.max():.3e}"

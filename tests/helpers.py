"""Shared helpers of the parity tests: seeded inputs, the oracle on subsets of rows/heads, and the tolerance.

Tolerance (stated by the build's target, calibrated on the reference's own tests: GPU flash vs f64 max abs 3e-3 in
tests/unit/test_backend_ggml.cpp:694): on f16 outputs, elementwise |got - ref| <= ATOL + RTOL * |ref| with ATOL = 2e-3,
RTOL = 1e-2, and per (row block, head) ||got - ref||_inf / ||ref||_inf <= 1e-2; natural-log LSE abs error <= 1e-3.
"""
import numpy as np

from oracle import oracle as O

ATOL = 2e-3
RTOL = 1e-2
LSE_ATOL = 1e-3


def normal_f16(rng, shape, sigma=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(np.float16)


def ref_attention(q, k, v, n_head, n_head_kv, hd, scale, p0=0, causal=True, rows=None, heads=None):
    """Oracle output for the selected query rows (absolute row indices) and query heads.

    Returns (out [len(rows)][len(heads)*hd], lse [len(rows)][len(heads)]) in float64. Rows and heads are restricted
    by slicing the inputs (one kv head at a time), which leaves the math of each (row, head) pair unchanged.
    """
    n_q = q.shape[0]
    rows = np.arange(n_q) if rows is None else np.asarray(rows)
    heads = np.arange(n_head) if heads is None else np.asarray(heads)
    G = n_head // n_head_kv
    out = np.zeros((len(rows), len(heads) * hd))
    lse = np.zeros((len(rows), len(heads)))
    for ri, t in enumerate(rows):
        n_vis = (p0 + t + 1) if causal else k.shape[0]
        kk, vv = k[:n_vis], v[:n_vis]
        for hi, h in enumerate(heads):
            g = h // G
            qs = q[t:t + 1, h * hd:(h + 1) * hd]
            o, l = O.attention_f64(qs, np.ascontiguousarray(kk[:, g * hd:(g + 1) * hd]),
                                   np.ascontiguousarray(vv[:, g * hd:(g + 1) * hd]), 1, 1, hd, scale,
                                   causal=False)
            out[ri, hi * hd:(hi + 1) * hd] = o[0]
            lse[ri, hi] = l[0, 0]
    return out, lse


def assert_close(got, ref, hd, what="", lse_got=None, lse_ref=None):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), (f"{what}: {bad.sum()} elements out of tolerance; max abs err {err.max():.3e} "
                           f"at {np.unravel_index(err.argmax(), err.shape)}")
    # per (row, head) relative inf-norm
    nh = got.shape[1] // hd
    e = err.reshape(got.shape[0], nh, hd).max(axis=2)
    r = np.abs(ref).reshape(got.shape[0], nh, hd).max(axis=2)
    rel = e / np.maximum(r, 1e-30)
    assert (rel <= RTOL).all(), f"{what}: max per-head relative error {rel.max():.3e}"
    if lse_got is not None:
        le = np.abs(np.asarray(lse_got, np.float64) - np.asarray(lse_ref, np.float64))
        assert le.max() <= LSE_ATOL, f"{what}: LSE max abs err {le.max():.3e}"
    return float(err.max())

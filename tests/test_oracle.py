"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it. CPU only.

Each check is chosen so that a plausible mistake in the oracle fails it:
  * torch's scaled_dot_product_attention in float64 (an independent library routine) with GQA, a causal mask with a
    chunk offset, and non-causal rows: catches a wrong GQA head mapping, a wrong causal limit or offset, a missing or
    misplaced scale, a transposed operand;
  * closed forms: scale 0 -> mean of the visible values (test_backend_ggml.cpp:715-735), one key -> that value, equal
    keys -> mean of the values, one dominant logit -> that value row;
  * invariants: GQA equals MHA over repeated key/value heads; a causal row equals a non-causal row over its prefix;
    the LSE equals log(sum(exp)) of the scores;
  * the committed golden fixtures (tests/golden, written by tests/golden/make_golden.py);
  * the f16 decoding routine against numpy on all 65536 bit patterns;
  * the restated reference CPU attention (cpu_attend_f32) against the f64 oracle within f32 error (the reference's CPU
    tolerance, test_backend_ggml.cpp:694: 2e-5), single- and multi-threaded bit-identical.
"""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
# the attention fixtures (the sa_* and lin_* files hold the self-attention and projection fixtures)
ATTN_FIXTURES = sorted(p for p in glob.glob(os.path.join(GOLDEN, "*.npz"))
                       if not os.path.basename(p).startswith(("sa_", "lin_")))


def rand_f16(rng, shape, sigma=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)).astype(np.float16)


def torch_sdpa(q, k, v, n_head, n_head_kv, hd, scale, p0, causal):
    n_q, n_kv = q.shape[0], k.shape[0]
    G = n_head // n_head_kv
    tq = torch.from_numpy(q.astype(np.float64)).view(n_q, n_head, hd).transpose(0, 1)
    tk = torch.from_numpy(k.astype(np.float64)).view(n_kv, n_head_kv, hd).transpose(0, 1)
    tv = torch.from_numpy(v.astype(np.float64)).view(n_kv, n_head_kv, hd).transpose(0, 1)
    mask = torch.ones(n_q, n_kv, dtype=torch.bool)
    if causal:
        mask = torch.arange(n_kv)[None, :] <= (p0 + torch.arange(n_q))[:, None]
    out = torch.nn.functional.scaled_dot_product_attention(tq[None], tk[None], tv[None], attn_mask=mask, scale=scale,
                                                           enable_gqa=G > 1)[0]
    s = scale * tq @ tk.repeat_interleave(G, dim=0).transpose(1, 2)
    lse = torch.logsumexp(s.masked_fill(~mask, float("-inf")), dim=-1)
    return out.transpose(0, 1).reshape(n_q, n_head * hd).numpy(), lse.transpose(0, 1).numpy()


@pytest.mark.parametrize("n_head,n_head_kv,hd,n_q,n_kv,p0,causal", [
    (14, 2, 64, 1, 40, 39, 1),      # decode row, G = 7
    (8, 2, 128, 12, 30, 18, 1),     # chunk at an offset, G = 4
    (4, 4, 64, 9, 9, 0, 1),         # MHA prompt
    (6, 3, 32, 5, 23, 0, 0),        # non-causal (cross-attention), G = 2
    (4, 1, 16, 7, 7, 0, 1),         # G = 4, one kv head
])
def test_oracle_matches_torch_sdpa_f64(n_head, n_head_kv, hd, n_q, n_kv, p0, causal):
    rng = np.random.default_rng(100 + n_head + n_q)
    q, k, v = rand_f16(rng, (n_q, n_head * hd)), rand_f16(rng, (n_kv, n_head_kv * hd)), rand_f16(rng, (n_kv, n_head_kv * hd))
    scale = 1.0 / np.sqrt(hd)
    out, lse = O.attention_f64(q, k, v, n_head, n_head_kv, hd, scale, p0=p0, causal=bool(causal))
    to, tl = torch_sdpa(q, k, v, n_head, n_head_kv, hd, scale, p0, causal)
    np.testing.assert_allclose(out, to, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, tl, rtol=0, atol=1e-12)


def test_scale_zero_is_mean_of_visible_values():
    rng = np.random.default_rng(1)
    n_q, n_kv, p0, hd = 6, 10, 4, 16
    q, k, v = rand_f16(rng, (n_q, 2 * hd)), rand_f16(rng, (n_kv, hd)), rand_f16(rng, (n_kv, hd))
    out, lse = O.attention_f64(q, k, v, 2, 1, hd, 0.0, p0=p0, causal=True)
    vd = v.astype(np.float64)
    for t in range(n_q):
        mean = vd[:p0 + t + 1].mean(axis=0)
        np.testing.assert_allclose(out[t, :hd], mean, atol=1e-14)
        np.testing.assert_allclose(out[t, hd:], mean, atol=1e-14)
        np.testing.assert_allclose(lse[t], np.log(p0 + t + 1), atol=1e-14)


def test_one_key_returns_that_value():
    rng = np.random.default_rng(2)
    q, k, v = rand_f16(rng, (1, 64)), rand_f16(rng, (1, 64)), rand_f16(rng, (1, 64))
    out, lse = O.attention_f64(q, k, v, 1, 1, 64, 0.125, causal=False)
    np.testing.assert_array_equal(out[0], v[0].astype(np.float64))
    np.testing.assert_allclose(lse[0, 0], 0.125 * float(np.dot(q[0].astype(np.float64), k[0].astype(np.float64))),
                               atol=1e-12)


def test_equal_keys_give_mean_of_values():
    rng = np.random.default_rng(3)
    k = np.tile(rand_f16(rng, (1, 32)), (9, 1))
    q, v = rand_f16(rng, (1, 32)), rand_f16(rng, (9, 32))
    out, _ = O.attention_f64(q, k, v, 1, 1, 32, 0.3, causal=False)
    np.testing.assert_allclose(out[0], v.astype(np.float64).mean(axis=0), atol=1e-14)


def test_dominant_logit_selects_its_value_row():
    hd = 16
    q = np.zeros((1, hd), np.float16)
    q[0, 0] = 60.0
    k = np.zeros((5, hd), np.float16)
    k[3, 0] = 60.0  # score 3600 * scale for key 3, 0 for the others
    v = np.arange(5 * hd, dtype=np.float16).reshape(5, hd)
    out, lse = O.attention_f64(q, k, v, 1, 1, hd, 1.0, causal=False)
    np.testing.assert_allclose(out[0], v[3].astype(np.float64), atol=1e-9)
    np.testing.assert_allclose(lse[0, 0], 3600.0, atol=1e-9)


def test_gqa_equals_mha_on_repeated_kv_heads():
    rng = np.random.default_rng(4)
    n_head, n_kv, hd, n_q, L = 12, 3, 32, 4, 25
    q, k, v = rand_f16(rng, (n_q, n_head * hd)), rand_f16(rng, (L, n_kv * hd)), rand_f16(rng, (L, n_kv * hd))
    G = n_head // n_kv
    # head h of the MHA problem reads kv head h // G: repeat each kv head G times, in order
    rep = lambda a: np.concatenate([np.tile(a[:, g * hd:(g + 1) * hd], (1, G)) for g in range(n_kv)], axis=1)
    a, la = O.attention_f64(q, k, v, n_head, n_kv, hd, 0.2, p0=L - n_q, causal=True)
    b, lb = O.attention_f64(q, rep(k), rep(v), n_head, n_head, hd, 0.2, p0=L - n_q, causal=True)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(la, lb)


def test_causal_row_is_noncausal_over_its_prefix():
    rng = np.random.default_rng(5)
    n_q, L, p0, hd = 5, 20, 15, 32
    q, k, v = rand_f16(rng, (n_q, 2 * hd)), rand_f16(rng, (L, 2 * hd)), rand_f16(rng, (L, 2 * hd))
    a, la = O.attention_f64(q, k, v, 2, 2, hd, 0.17, p0=p0, causal=True)
    for t in range(n_q):
        b, lb = O.attention_f64(q[t:t + 1], k[:p0 + t + 1], v[:p0 + t + 1], 2, 2, hd, 0.17, causal=False)
        np.testing.assert_array_equal(a[t], b[0])
        np.testing.assert_array_equal(la[t], lb[0])


def test_lse_is_log_sum_exp_of_scores():
    rng = np.random.default_rng(6)
    q, k, v = rand_f16(rng, (1, 64)), rand_f16(rng, (50, 64)), rand_f16(rng, (50, 64))
    _, lse = O.attention_f64(q, k, v, 1, 1, 64, 0.125, causal=False)
    s = 0.125 * k.astype(np.float64) @ q[0].astype(np.float64)
    np.testing.assert_allclose(lse[0, 0], np.log(np.exp(s).sum()), rtol=1e-13)


def test_oracle_rejects_bad_shapes():
    q = np.zeros((1, 64), np.float16)
    with pytest.raises(ValueError):
        O.attention_f64(q, q, q, 3, 2, 32, 1.0)  # 3 % 2 != 0


def test_f16_decoding_matches_numpy_on_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = O.f16_to_f32(bits.view(np.float16))
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


@pytest.mark.parametrize("path", ATTN_FIXTURES, ids=os.path.basename)
def test_golden_fixture(path):
    z = np.load(path)
    n_head, n_head_kv, hd, n_q, n_kv, p0, causal = (int(x) for x in z["meta"])
    out, lse = O.attention_f64(z["q"], z["k"], z["v"], n_head, n_head_kv, hd, float(z["scale"]), p0=p0,
                               causal=bool(causal), n_kv=n_kv)
    np.testing.assert_allclose(out, z["out"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, z["lse"], rtol=0, atol=1e-12)
    to, tl = torch_sdpa(z["q"], z["k"], z["v"], n_head, n_head_kv, hd, float(z["scale"]), p0, causal)
    np.testing.assert_allclose(z["out"], to, rtol=0, atol=1e-12)


def test_golden_fixtures_present():
    assert len(ATTN_FIXTURES) >= 7
    assert len(glob.glob(os.path.join(GOLDEN, "sa_*.npz"))) >= 5 and len(glob.glob(os.path.join(GOLDEN, "lin_*.npz"))) >= 3


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "sa_*.npz"))), ids=os.path.basename)
def test_golden_self_attention_fixture(path):
    z = np.load(path)
    y = O.self_attention_f64(z["qkv"], int(z["heads"]), float(z["scale"]))
    np.testing.assert_allclose(y, z["y"], rtol=0, atol=1e-12)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "lin_*.npz"))), ids=os.path.basename)
def test_golden_linear_fixture(path):
    z = np.load(path)
    flags = int(z["flags"])
    y = O.linear_f64(z["x"], z["w"], flags=flags, half_input=z["x"].shape[0] > 8, eps=float(z["eps"]),
                     gamma=z["gamma"] if flags & 1 else None, bias=z["bias"] if flags & 4 else None)
    np.testing.assert_allclose(y, z["y"], rtol=0, atol=1e-12)


@pytest.mark.parametrize("causal", [0, 1])
def test_cpu_restatement_within_f32_error(causal):
    rng = np.random.default_rng(7)
    n_head, n_kv, hd, n_q, L = 8, 2, 64, 6, 300
    q, k, v = rand_f16(rng, (n_q, n_head * hd)), rand_f16(rng, (L, n_kv * hd)), rand_f16(rng, (L, n_kv * hd))
    scale = 1.0 / np.sqrt(hd)
    ref, _ = O.attention_f64(q, k, v, n_head, n_kv, hd, scale, p0=L - n_q, causal=bool(causal))
    got = O.cpu_attend_f32(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), n_head, n_kv, hd, scale,
                           p0=L - n_q, causal=bool(causal))
    assert np.abs(got - ref).max() < 2e-5
    got4 = O.cpu_attend_f32(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), n_head, n_kv, hd, scale,
                            p0=L - n_q, causal=bool(causal), n_threads=4)
    np.testing.assert_array_equal(got, got4)


# ---- rotary embedding (oracle_rope_f32) ----

def _rope_double(x, mode, base, hd, pos):
    """The reference test's own rope in double (tests/unit/test_metal_llama_decoder.cpp:180-189)."""
    y = np.array(x, dtype=np.float64)
    for i in range(hd // 2):
        th = pos * (float(base) ** (-2.0 * i / hd))
        i0, i1 = (i, i + hd // 2) if mode == 1 else (2 * i, 2 * i + 1)
        a, b = y[..., i0].copy(), y[..., i1].copy()
        y[..., i0] = a * np.cos(th) - b * np.sin(th)
        y[..., i1] = a * np.sin(th) + b * np.cos(th)
    return y


@pytest.mark.parametrize("mode,base,hd", [(0, 500000.0, 128), (1, 1000000.0, 64), (0, 10000.0, 64), (1, 10000.0, 128)])
@pytest.mark.parametrize("pos", [0, 1, 7, 513, 8191, 32767])
def test_rope_matches_reference_double_rope(mode, base, hd, pos):
    rng = np.random.default_rng(pos + hd)
    x = rng.standard_normal((5, hd)).astype(np.float32)
    got = O.rope_f32(x, mode, base, hd, pos)
    ref = _rope_double(x, mode, base, hd, pos)
    # the oracle's angle is an f32 product: off by at most ~1.5 f32 ulps of theta <= pos, which moves a pair of norm r
    # by r * |d theta|; plus the final f32 rounding
    r = np.sqrt(x.astype(np.float64) ** 2).max() * np.sqrt(2)
    tol = r * (pos * 2.0 ** -23 * 1.5 + 1e-12) + 2e-7 * np.abs(ref).max()
    assert np.abs(got - ref).max() <= tol
    if pos == 0:
        assert np.array_equal(got, x)


def test_rope_mode2_is_identity_and_pairs_keep_their_norm():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    assert np.array_equal(O.rope_f32(x, 2, 10000.0, 128, 999), x)
    for mode in (0, 1):
        y = O.rope_f32(x, mode, 10000.0, 128, 4321).astype(np.float64)
        xd = x.astype(np.float64)
        if mode == 0:
            n0, n1 = xd[:, 0::2] ** 2 + xd[:, 1::2] ** 2, y[:, 0::2] ** 2 + y[:, 1::2] ** 2
        else:
            n0, n1 = xd[:, :64] ** 2 + xd[:, 64:] ** 2, y[:, :64] ** 2 + y[:, 64:] ** 2
        np.testing.assert_allclose(n1, n0, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("mode", [0, 1])
def test_rope_relative_position_property(mode):
    # <R(m) q, R(n) k> = <R(m - n) q, k>: what makes rotary embedding positional; a wrong pair, sign or frequency
    # index between q and k breaks it
    rng = np.random.default_rng(11)
    q, k = rng.standard_normal((2, 64)).astype(np.float32)
    for m, n in [(100, 37), (2000, 1999), (777, 0)]:
        a = np.dot(O.rope_f32(q, mode, 10000.0, 64, m).astype(np.float64), O.rope_f32(k, mode, 10000.0, 64, n))
        b = np.dot(O.rope_f32(q, mode, 10000.0, 64, m - n).astype(np.float64), k.astype(np.float64))
        assert abs(a - b) <= 1e-4 * (1 + abs(b)) + 64 * m * 2.0 ** -23


def test_rope_neox_is_adjacent_under_the_half_interleave_permutation():
    rng = np.random.default_rng(5)
    hd = 128
    x = rng.standard_normal((3, hd)).astype(np.float32)
    perm = np.empty(hd, dtype=np.int64)  # adjacent position 2i <- half position i, 2i+1 <- i + hd/2
    perm[0::2] = np.arange(hd // 2)
    perm[1::2] = np.arange(hd // 2) + hd // 2
    a = O.rope_f32(x[:, perm], 0, 10000.0, hd, 1234)
    b = O.rope_f32(x, 1, 10000.0, hd, 1234)[:, perm]
    assert np.array_equal(a, b)


# ---- binary16 rounding and the projections (oracle_f32_to_f16, oracle_linear_f64) ----

def test_f32_to_f16_matches_numpy_round_to_nearest_even():
    rng = np.random.default_rng(21)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * np.float32(s) for s in (1e-6, 1e-3, 1, 300, 6e4)])
    specials = np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 1e9, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25,
                         3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11],
                        dtype=np.float32)
    x = np.concatenate([x, specials])
    np.testing.assert_array_equal(O.f32_to_f16(x).view(np.uint16), x.astype(np.float16).view(np.uint16))


def _lin_inputs(rng, M, N, K):
    x = rng.standard_normal((M, K), dtype=np.float32) * 3
    w = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    return x, w, g, b


@pytest.mark.parametrize("half_input", [False, True])
def test_linear_matches_numpy(half_input):
    rng = np.random.default_rng(22)
    x, w, g, b = _lin_inputs(rng, 5, 40, 64)
    eps = 1e-5
    scale = (1 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1) + eps)).astype(np.float32)
    if half_input:
        a = (x * (g[None, :] * scale[:, None])).astype(np.float16).astype(np.float64)
        ref = a @ w.astype(np.float64).T + b
    else:
        a = (x * g[None, :]).astype(np.float64)
        ref = (a @ w.astype(np.float64).T) * scale[:, None].astype(np.float64) + b
    got = O.linear_f64(x, w, flags=1 | 4, half_input=half_input, eps=eps, gamma=g, bias=b)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    # plain product (no norm): half_input rounds x to half, the matvec form keeps it
    got = O.linear_f64(x, w, half_input=half_input)
    xa = x.astype(np.float16) if half_input else x
    np.testing.assert_allclose(got, xa.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-12, atol=1e-12)


def test_linear_closed_forms():
    rng = np.random.default_rng(23)
    K = 32
    x = rng.standard_normal((3, K)).astype(np.float32)
    eye = np.eye(K, dtype=np.float16)
    np.testing.assert_array_equal(O.linear_f64(x, eye), x.astype(np.float64))           # W = I: y = x
    b = rng.standard_normal(K).astype(np.float32)
    np.testing.assert_array_equal(O.linear_f64(x, np.zeros((K, K), np.float16), flags=4, bias=b),
                                  np.broadcast_to(b.astype(np.float64), (3, K)))         # W = 0: y = bias
    y0 = rng.standard_normal((3, K))
    np.testing.assert_allclose(O.linear_f64(x, eye, flags=2, y0=y0), y0 + x, rtol=0, atol=1e-15)  # residual add
    c = np.full((1, K), 2.5, np.float32)  # constant row: scale = 1 / sqrt(c^2 + eps), gamma = 1 -> y = c * scale
    got = O.linear_f64(c, eye, flags=1, eps=1e-6, gamma=np.ones(K, np.float32))
    np.testing.assert_allclose(got, np.float32(1 / np.sqrt(2.5 ** 2 + 1e-6)) * 2.5, rtol=1e-7)


# ---- the IR SelfAttention oracle (packed [B, N, 3E] rows, no mask) ----

@pytest.mark.parametrize("B,N,H,D", [(1, 5, 2, 4), (2, 7, 3, 8), (1, 1, 1, 16), (1, 17, 4, 64), (1, 9, 2, 6),
                                     (1, 40, 4, 80)])
def test_self_attention_oracle_matches_torch_and_the_c_oracle(B, N, H, D):
    """The reference's own test shapes (kAttnCases, test_backend_ggml.cpp:679-681, ViT-H reduced to 40 tokens): the
    numpy restatement against torch SDPA in float64 and against oracle_attention_f64 (C) on f16-representable inputs."""
    rng = np.random.default_rng(700 + N)
    E = H * D
    qkv = rand_f16(rng, (B, N, 3 * E))
    scale = D ** -0.5
    y = O.self_attention_f64(qkv, H, scale)
    x = torch.from_numpy(qkv.astype(np.float64))
    q, k, v = (x[..., i * E:(i + 1) * E].reshape(B, N, H, D).transpose(1, 2) for i in range(3))
    t = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=scale).transpose(1, 2).reshape(B, N, E)
    np.testing.assert_allclose(y, t.numpy(), rtol=0, atol=1e-12)
    for b in range(B):
        o, _ = O.attention_f64(qkv[b, :, :E], np.ascontiguousarray(qkv[b, :, E:2 * E]),
                               np.ascontiguousarray(qkv[b, :, 2 * E:]), H, H, D, scale, causal=False)
        np.testing.assert_allclose(y[b], o, rtol=0, atol=1e-12)


def test_self_attention_oracle_closed_forms():
    """scale 0 -> every row is the mean of v over the tokens (test_backend_ggml.cpp:715-735); one token -> its v;
    batch elements are independent (swapping them swaps the outputs)."""
    rng = np.random.default_rng(710)
    B, N, H, D = 2, 6, 2, 8
    E = H * D
    qkv = rng.standard_normal((B, N, 3 * E))
    y = O.self_attention_f64(qkv, H, 0.0)
    np.testing.assert_allclose(y, np.broadcast_to(qkv[:, :, 2 * E:].mean(axis=1, keepdims=True), y.shape), atol=1e-14)
    one = O.self_attention_f64(qkv[:, :1], H, 0.7)
    np.testing.assert_allclose(one[:, 0], qkv[:, 0, 2 * E:], atol=1e-14)
    np.testing.assert_allclose(O.self_attention_f64(qkv[::-1], H, 0.3), O.self_attention_f64(qkv, H, 0.3)[::-1],
                               atol=1e-14)


def test_oracle_under_address_and_undefined_behaviour_sanitizers():
    # every oracle function on small cases with exactly sized buffers, built with -fsanitize=address,undefined
    # (oracle/sanitize_check.c); any out-of-bounds access, leak or undefined arithmetic fails the run
    import subprocess
    r = subprocess.run(["make", "-s", "-C", os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"), "sanitize"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "sanitize_check: ok" in r.stdout

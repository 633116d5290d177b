"""Writes the golden fixtures of the attention hot path (tests/golden/*.npz).

The reference (dooms.cpp 0.6.1) holds no golden vectors for this path: its tests draw random inputs from std::mt19937
seeds and compare against references written in the tests (tests/unit/test_metal_llama_decoder.cpp:110-192,
tests/unit/test_backend_ggml.cpp:650-675). These fixtures are small inputs from numpy's PCG64 generator (bit-identical on
every machine with this numpy) and the expected outputs of the f64 oracle (oracle/oracle.c), each checked at generation
time against torch's scaled_dot_product_attention in float64, an independent library routine. Inputs are f16 bit
patterns; outputs f64; lse is the natural-log log-sum-exp of the scaled masked scores.

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

# name: (n_head, n_head_kv, hd, n_q, n_kv, p0, causal, scale or None, seed, sigma)
CASES = {
    "decode_qwen05b_g7_hd64": (14, 2, 64, 1, 37, 36, 1, None, 11, 1.0),
    "prefill_gqa4_hd128_chunk": (8, 2, 128, 9, 21, 12, 1, None, 12, 0.5),
    "prefill_mha_hd64_full": (3, 3, 64, 17, 17, 0, 1, None, 13, 1.0),
    "cross_beam5_mha_hd64": (4, 4, 64, 5, 29, 0, 0, None, 14, 1.0),
    "whisper_prompt_rows_hd64": (2, 2, 64, 8, 19, 11, 1, None, 15, 1.0),
    "scale0_uniform_hd64": (2, 1, 64, 3, 10, 7, 1, 0.0, 16, 1.0),
    "decode_llama3_g4_hd128": (8, 2, 128, 1, 130, 129, 1, None, 17, 1.0),
}


def make_case(n_head, n_head_kv, hd, n_q, n_kv, p0, causal, scale, seed, sigma):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((n_q, n_head * hd), dtype=np.float32) * np.float32(sigma)).astype(np.float16)
    k = (rng.standard_normal((n_kv, n_head_kv * hd), dtype=np.float32) * np.float32(sigma)).astype(np.float16)
    v = (rng.standard_normal((n_kv, n_head_kv * hd), dtype=np.float32) * np.float32(sigma)).astype(np.float16)
    sc = 1.0 / np.sqrt(hd) if scale is None else scale
    out, lse = O.attention_f64(q, k, v, n_head, n_head_kv, hd, sc, p0=p0, causal=bool(causal), n_kv=n_kv)
    return dict(q=q, k=k, v=v, out=out, lse=lse,
                meta=np.array([n_head, n_head_kv, hd, n_q, n_kv, p0, causal], np.int64), scale=np.float64(sc))


def torch_reference(case):
    """softmax(scale q k^T + mask) v and the row LSE through torch (float64), independent of the oracle."""
    import torch
    n_head, n_head_kv, hd, n_q, n_kv, p0, causal = (int(x) for x in case["meta"])
    G = n_head // n_head_kv
    q = torch.from_numpy(case["q"].astype(np.float64)).view(n_q, n_head, hd).transpose(0, 1)
    k = torch.from_numpy(case["k"].astype(np.float64)).view(n_kv, n_head_kv, hd).transpose(0, 1)
    v = torch.from_numpy(case["v"].astype(np.float64)).view(n_kv, n_head_kv, hd).transpose(0, 1)
    mask = torch.ones(n_q, n_kv, dtype=torch.bool)
    if causal:
        mask = torch.arange(n_kv)[None, :] <= (p0 + torch.arange(n_q))[:, None]
    out = torch.nn.functional.scaled_dot_product_attention(q[None], k[None], v[None], attn_mask=mask,
                                                           scale=float(case["scale"]), enable_gqa=G > 1)[0]
    kk = k.repeat_interleave(G, dim=0)
    s = float(case["scale"]) * q @ kk.transpose(1, 2)
    s = s.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    return out.transpose(0, 1).reshape(n_q, n_head * hd).numpy(), lse.transpose(0, 1).numpy()


# IR SelfAttention (sa_*): the reference's own test shapes (kAttnCases, tests/unit/test_backend_ggml.cpp:679-681),
# packed [B, N, 3E] rows in f16, U(-1, 1) like the reference's rnd(); name: (B, N, heads, head_dim, seed)
SA_CASES = {
    "sa_b1_n5_h2_d4": (1, 5, 2, 4, 705),
    "sa_b2_n7_h3_d8": (2, 7, 3, 8, 707),
    "sa_b1_n9_h2_d6": (1, 9, 2, 6, 709),
    "sa_b1_n17_h4_d64": (1, 17, 4, 64, 717),
    "sa_b1_n40_h2_d80": (1, 40, 2, 80, 740),
}

# projections (lin_*): x f32 [M][K], w f16 [N][K], gamma, bias; name: (M, N, K, flags, seed). M <= 8 is the f32-input
# GEMV form, M > 8 the half-staged GEMM form (llama_kernels.h:96-126, 186-199)
LIN_CASES = {
    "lin_gemv_m3_norm_bias": (3, 40, 64, 1 | 4, 31),
    "lin_gemm_m20_norm_bias": (20, 48, 96, 1 | 4, 32),
    "lin_gemm_m12_plain": (12, 24, 160, 0, 33),
}


def make_sa_case(B, N, H, D, seed):
    import torch
    rng = np.random.default_rng(seed)
    E = H * D
    qkv = rng.uniform(-1, 1, (B, N, 3 * E)).astype(np.float16)
    scale = D ** -0.5
    y = O.self_attention_f64(qkv, H, scale)
    x = torch.from_numpy(qkv.astype(np.float64))
    q, k, v = (x[..., i * E:(i + 1) * E].reshape(B, N, H, D).transpose(1, 2) for i in range(3))
    t = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=scale).transpose(1, 2).reshape(B, N, E)
    assert np.abs(t.numpy() - y).max() < 1e-12
    return dict(qkv=qkv, y=y, heads=np.int64(H), scale=np.float64(scale))


def make_lin_case(M, N, K, flags, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, K), dtype=np.float32) * 2).astype(np.float32)
    w = (rng.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float16)
    g = rng.uniform(0.2, 2.0, K).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    eps = 1e-5
    half_input = M > 8
    y = O.linear_f64(x, w, flags=flags, half_input=half_input, eps=eps, gamma=g if flags & 1 else None,
                     bias=b if flags & 4 else None)
    # independent restatement in numpy (the two staging forms of the reference)
    xs = x.astype(np.float64)
    scale = (1 / np.sqrt((xs ** 2).mean(axis=1) + eps)).astype(np.float32)
    if half_input:
        a = (x * (g[None, :] * scale[:, None])).astype(np.float16) if flags & 1 else x.astype(np.float16)
        ref = a.astype(np.float64) @ w.astype(np.float64).T
    else:
        a = (x * g[None, :]).astype(np.float64) if flags & 1 else xs
        ref = a @ w.astype(np.float64).T
        if flags & 1:
            ref = ref * scale[:, None].astype(np.float64)
    if flags & 4:
        ref = ref + b
    assert np.abs(ref - y).max() < 1e-9
    return dict(x=x, w=w, gamma=g, bias=b, y=y, flags=np.int64(flags), eps=np.float64(eps))


def main():
    for name, args in CASES.items():
        c = make_case(*args)
        to, tl = torch_reference(c)
        assert np.abs(to - c["out"]).max() < 1e-12, name
        assert np.abs(tl - c["lse"]).max() < 1e-12, name
        np.savez(os.path.join(HERE, name + ".npz"), **c)
        print(name, c["out"].shape)
    for name, args in SA_CASES.items():
        c = make_sa_case(*args)
        np.savez(os.path.join(HERE, name + ".npz"), **c)
        print(name, c["y"].shape)
    for name, args in LIN_CASES.items():
        c = make_lin_case(*args)
        np.savez(os.path.join(HERE, name + ".npz"), **c)
        print(name, c["y"].shape)


if __name__ == "__main__":
    main()

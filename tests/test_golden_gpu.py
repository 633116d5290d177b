"""The committed golden fixtures (tests/golden/*.npz) through the HIP entry points, against the fixture outputs: the
attention fixtures through mx_attn_prefill and mx_attn_decode, sa_* through mx_self_attention (f16 rows, and the same
values as f32 rows), lin_* through mx_linear."""
import glob
import os

import numpy as np
import pytest
import torch

from dooms_amd import attention as A
from helpers import assert_close

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(p for p in glob.glob(os.path.join(GOLDEN, "*.npz"))
                  if not os.path.basename(p).startswith(("sa_", "lin_")))
SA_FIXTURES = sorted(glob.glob(os.path.join(GOLDEN, "sa_*.npz")))
LIN_FIXTURES = sorted(glob.glob(os.path.join(GOLDEN, "lin_*.npz")))


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_fixture_prefill(device, path):
    z = np.load(path)
    n_head, n_head_kv, hd, n_q, n_kv, p0, causal = (int(x) for x in z["meta"])
    q, k, v = (torch.from_numpy(z[n]).to(device) for n in ("q", "k", "v"))
    out, lse = A.prefill(q, k, v, n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, p0=p0, n_kv=n_kv,
                         causal=bool(causal), scale=float(z["scale"]), want_lse=True)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), z["out"], hd, os.path.basename(path), lse.cpu().numpy(), z["lse"])


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_fixture_decode(device, path):
    z = np.load(path)
    n_head, n_head_kv, hd, n_q, n_kv, p0, causal = (int(x) for x in z["meta"])
    if causal and p0 != n_kv - n_q:
        pytest.skip("decode rows sit at the end of the cache")
    q, k, v = (torch.from_numpy(z[n]).to(device) for n in ("q", "k", "v"))
    out, lse = A.decode(q, [k], [v], [n_kv], n_head=n_head, n_head_kv=n_head_kv, head_dim=hd, n_q=n_q,
                        causal=bool(causal), scale=float(z["scale"]), want_lse=True)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), z["out"], hd, os.path.basename(path), lse.cpu().numpy(), z["lse"])


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("path", SA_FIXTURES, ids=os.path.basename)
def test_fixture_self_attention(device, path, dtype):
    z = np.load(path)
    H = int(z["heads"])
    B, N, E3 = z["qkv"].shape
    qkv = torch.from_numpy(z["qkv"]).to(device).to(dtype)
    y = A.self_attention(qkv, heads=H, scale=float(z["scale"]))
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().reshape(B * N, E3 // 3)
    assert_close(got, z["y"].reshape(B * N, E3 // 3), (E3 // 3) // H, os.path.basename(path))


@pytest.mark.parametrize("path", LIN_FIXTURES, ids=os.path.basename)
def test_fixture_linear(device, path):
    z = np.load(path)
    flags = int(z["flags"])
    x = torch.from_numpy(z["x"]).to(device)
    w = torch.from_numpy(z["w"]).to(device)
    y = A.linear(x, w, gamma=torch.from_numpy(z["gamma"]).to(device) if flags & 1 else None,
                 bias=torch.from_numpy(z["bias"]).to(device) if flags & 4 else None, eps=float(z["eps"]))
    torch.cuda.synchronize()
    ref = z["y"]
    # f32 accumulation of the oracle's operands: |err| <= 2^-10 sum |a w| (+1e-6); the operand sums bound that by
    # 2^-10 * K * max|a| * max|w| (see tests/test_linear_gpu.py for the per-element form)
    K = z["x"].shape[1]
    bound = 2.0 ** -10 * K * np.abs(z["x"]).max() * 2 * np.abs(z["w"].astype(np.float64)).max() + 1e-6
    assert np.abs(y.cpu().numpy() - ref).max() <= bound

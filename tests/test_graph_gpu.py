"""Both entry points captured in a HIP graph and replayed several times, with eager work and synchronizations in
between: every replay must equal the eager result bit for bit (the decode kernel keeps split counters in its workspace;
they must be back at zero after every replay)."""
import numpy as np
import pytest
import torch

from dooms_amd import attention as A
from helpers import normal_f16

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(device):
    rng = np.random.default_rng(90)
    L, hd = 5000, 128
    q = torch.from_numpy(normal_f16(rng, (1, 32 * hd))).to(device)
    k = torch.from_numpy(normal_f16(rng, (L, 8 * hd))).to(device)
    v = torch.from_numpy(normal_f16(rng, (L, 8 * hd))).to(device)
    pq = torch.from_numpy(normal_f16(rng, (300, 28 * hd))).to(device)
    pk = torch.from_numpy(normal_f16(rng, (300, 4 * hd))).to(device)
    pv = torch.from_numpy(normal_f16(rng, (300, 4 * hd))).to(device)
    ws = A.new_workspace(A.decode_workspace_bytes(n_head=32, n_head_kv=8, head_dim=hd, n_q=1, batch=1, max_kv_len=L),
                         device)
    d_out = torch.empty(1, 32 * hd, dtype=torch.float16, device=device)
    p_out = torch.empty(300, 28 * hd, dtype=torch.float16, device=device)

    def step():
        A.decode(q, [k], [v], [L], n_head=32, n_head_kv=8, head_dim=hd, out=d_out, workspace=ws)
        A.prefill(pq, pk, pv, n_head=28, n_head_kv=4, head_dim=hd, out=p_out)

    step()
    torch.cuda.synchronize()
    ref_d, ref_p = d_out.clone(), p_out.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(5):
        d_out.zero_()
        p_out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(d_out, ref_d), f"decode replay {i}"
        assert torch.equal(p_out, ref_p), f"prefill replay {i}"
        step()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(d_out, ref_d)


def test_graph_replays_linear_and_self_attention(device):
    """The projections (GEMV row, staged GEMM chunk through mx_linear's hand-written kernels) and the IR
    self-attention in all three workspace modes, captured together: nothing recorded may change the result on later
    replays."""
    rng = np.random.default_rng(91)
    K, N = 512, 384
    w = torch.from_numpy(normal_f16(rng, (N, K), 0.05)).to(device)
    gamma = torch.from_numpy(rng.uniform(0.5, 1.5, K).astype(np.float32)).to(device)
    bias = torch.from_numpy(rng.normal(0, 1, N).astype(np.float32)).to(device)
    x1 = torch.from_numpy(rng.normal(0, 1, (1, K)).astype(np.float32)).to(device)
    xm = torch.from_numpy(rng.normal(0, 1, (200, K)).astype(np.float32)).to(device)
    y1 = torch.empty(1, N, dtype=torch.float32, device=device)
    ym = torch.empty(200, N, dtype=torch.float32, device=device)
    sa = {
        "f16_hd64": torch.from_numpy(normal_f16(rng, (2, 150, 3 * 256))).to(device),
        "f32_hd128": torch.from_numpy(rng.normal(0, 1, (1, 97, 3 * 512)).astype(np.float32)).to(device),
        "bf16_hd80": torch.from_numpy(rng.normal(0, 1, (3, 40, 3 * 160)).astype(np.float32)).to(device)
        .to(torch.bfloat16),
    }
    heads = {"f16_hd64": 4, "f32_hd128": 4, "bf16_hd80": 2}
    sa_out = {k: torch.empty(v.shape[0], v.shape[1], v.shape[2] // 3, dtype=v.dtype, device=device)
              for k, v in sa.items()}

    def step():
        A.linear(x1, w, out=y1, gamma=gamma, bias=bias)
        A.linear(xm, w, out=ym, gamma=gamma, bias=bias)
        for name, qkv in sa.items():
            A.self_attention(qkv, heads=heads[name], out=sa_out[name])

    outs = [y1, ym] + list(sa_out.values())
    step()
    torch.cuda.synchronize()
    refs = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    names = ["gemv", "gemm"] + list(sa_out)
    for i in range(4):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for name, o, r in zip(names, outs, refs):
            assert torch.equal(o, r), f"{name} replay {i}"
        step()
        torch.cuda.synchronize()
        for name, o, r in zip(names, outs, refs):
            assert torch.equal(o, r), f"{name} eager after replay {i}"

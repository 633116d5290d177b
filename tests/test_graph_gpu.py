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

#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X: prints ONE JSON line.

Headline (value): decode attention at the Llama-3-8B shape (32 q / 8 kv heads, head_dim 128, batch 1, 8192-token f16
KV cache). One step = the decode attention of all 32 layers, each layer with its own K/V buffers (32 x 33.6 MB = 1.07 GB,
well past the 256 MB Infinity Cache, so every step streams K/V from HBM). value = algorithmic bytes / time in GB/s.

Beside it (same JSON line): prefill TFLOP/s on the Qwen2.5-7B 32k-token causal prompt in 2048-query chunks, the other
BASELINE configurations, a same-run streaming-copy bandwidth, and the reference's CPU attention (restated in
oracle/oracle.c) timed on this host's cores on a bounded sample.

Timing: every figure replays a HIP graph of one step (the decode step is 32 launches of a few microseconds, too short
to issue from Python one by one); K steps are bracketed by synchronize() on both sides and timed with events on the
stream the kernels run on. The roofline's per-launch duration is that timed region divided by the launches in it
(so it includes the gaps between back-to-back launches); rocprofv3's kernel durations for the same command are in
profiles/. HBM traffic per launch comes from rocprofv3 --pmc runs recorded in profiles/traffic.json.

Algorithmic work (what `achieved` divides):
  decode bytes per (sequence, layer) = 2 * L * n_kv * hd * 2 (K+V, f16, each byte once) + 2 * n_head * hd * 2 (Q, O)
  prefill FLOPs per head = 4 * hd * (unmasked (query, key) pairs); a chunk of M rows at offset p0 has M p0 + M(M+1)/2.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
F16_PEAK_TFLOPS = 2500.0   # MI355X dense f16 MFMA
METRIC = "decode-attn achieved HBM GB/s + prefill-attn TFLOP/s (fraction of peak)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget per leg")
    ap.add_argument("--only", choices=["decode", "prefill", "all", "decode-headline", "prefill-headline", "linear",
                                       "self-attention"], default="all",
                    help="*-headline: only the headline workload of that path (for profiling one kernel)")
    ap.add_argument("--summarize", metavar="CSV",
                    help="no GPU work: summarize a rocprofv3 kernel_trace.csv (durations) or counter_collection.csv "
                         "(counters) over the last --last dispatches of the kernels whose names contain --kernel")
    ap.add_argument("--kernel", default="decode_kernel")
    ap.add_argument("--last", type=int, default=0, help="dispatches at the end of the trace to summarize (0: all)")
    ap.add_argument("--per-dispatch", action="store_true",
                    help="with --summarize on a counter_collection.csv: one row per dispatch (duration, shader clock "
                         "from GRBM_GUI_ACTIVE, MFMA busy per SIMD, and each SQ_ counter per SQ_WAVE_CYCLES)")
    ap.add_argument("--trace-decode", action="store_true",
                    help="phase timestamps of the decode kernel (dooms_amd/libmx_attn_trace.so) on the headline and "
                         "short-shape workloads: one JSON line per workload, microseconds from the launch's first start")
    return ap.parse_args()


def summarize(path, kernel, last, per_dispatch=False):
    """The timed region of a profiled bench.py run is its last dispatches (graph replays after the warmup), so a
    summary over the last `last` dispatches of `kernel` reconciles with the ms_per_step the same run printed.
    Prints a text summary: durations (kernel trace) or per-dispatch counter averages (counter collection), and for
    counters also what the same counters read for the run's 1 GiB copy kernel (the scale of FETCH_SIZE/WRITE_SIZE)."""
    import csv
    from collections import OrderedDict
    with open(path, newline="") as f:
        rows = list(csv.DictReader(f))
    if "Counter_Name" in rows[0]:
        disp = OrderedDict()
        for r in rows:
            disp.setdefault((r["Dispatch_Id"], r["Kernel_Name"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
        sel = [(k, v) for k, v in disp.items() if kernel in k[1]]
        sel = sel[-last:] if last else sel
        copies = [v for k, v in disp.items() if "copyBuffer" in k[1]]
        print(f"kernel: {sel[0][0][1][:120]}")
        print(f"dispatches summarized: {len(sel)} (the last {last or 'all'} of {sum(kernel in k[1] for k in disp)})")
        for c in sel[0][1]:
            vals = [v[c] for _, v in sel]
            print(f"  {c}: avg {sum(vals) / len(vals):.2f}  min {min(vals):.2f}  max {max(vals):.2f}")
        ts = {}
        for r in rows:
            if "Start_Timestamp" in r and "End_Timestamp" in r:
                ts[(r["Dispatch_Id"], r["Kernel_Name"])] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        if per_dispatch and ts:
            # clock = GRBM_GUI_ACTIVE / 8 XCDs / duration; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / the
            # cycles per XCD; other SQ_ counters as fractions of SQ_WAVE_CYCLES
            names = [c for c in sel[0][1] if c.startswith("SQ_") and c not in ("SQ_WAVE_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES")]
            print("dispatch | duration us | clock GHz | MFMA busy | " + " | ".join(n.lower() for n in names))
            for k, v in sel:
                ns = ts[k]
                cyc = v.get("GRBM_GUI_ACTIVE", 0.0) / 8
                row = [k[0], f"{ns / 1e3:.1f}", f"{cyc / ns:.2f}" if cyc else "-",
                       f"{v['SQ_VALU_MFMA_BUSY_CYCLES'] / 1024 / cyc:.2f}" if cyc and "SQ_VALU_MFMA_BUSY_CYCLES" in v else "-"]
                wc = v.get("SQ_WAVE_CYCLES")
                row += [f"{v[n] / wc:.3f}" if wc else f"{v[n]:.0f}" for n in names]
                print(" | ".join(row))
        if "GRBM_GUI_ACTIVE" in sel[0][1] and ts:
            # GRBM_GUI_ACTIVE sums the busy cycles of the 8 XCDs: cycles per XCD / duration is the shader clock
            cyc = sum(v["GRBM_GUI_ACTIVE"] / 8 for _, v in sel)
            ns = sum(ts[k] for k, _ in sel)
            print(f"  clock over the summarized dispatches (GRBM_GUI_ACTIVE / 8 / duration): {cyc / ns:.3f} GHz")
        if copies:
            for c in copies[-1]:
                print(f"  copyBuffer (1 GiB copy of the same run) {c}: {copies[-1][c]:.2f}")
        return 0
    sel = [r for r in rows if kernel in r["Kernel_Name"]]
    n_all = len(sel)
    sel = sel[-last:] if last else sel
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in sel]  # us
    span = (int(sel[-1]["End_Timestamp"]) - int(sel[0]["Start_Timestamp"])) / 1e3
    names = sorted({r["Kernel_Name"][:120] for r in sel})
    print(f"kernel: {'; '.join(names)}")
    print(f"dispatches summarized: {len(sel)} (the last {last or 'all'} of {n_all})")
    print(f"duration us: avg {sum(dur) / len(dur):.3f}  min {min(dur):.3f}  max {max(dur):.3f}  sum {sum(dur):.1f}")
    print(f"first start to last end: {span:.1f} us")
    return 0


def time_graph(torch, step, steps, warmup):
    """Captures step() into a HIP graph and returns ms per replay over `steps` replays (after `warmup`)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # eager once on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps, g


def measured_traffic(key):
    """HBM bytes per launch of a headline kernel as measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs and
    committed in profiles/traffic.json (with the commands and the copy-kernel scale factors), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)["workloads"][key]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def measured_clock(key):
    """The shader clock (GHz) that a rocprofv3 --pmc GRBM_GUI_ACTIVE run measured over a headline kernel's timed
    dispatches, as committed in profiles/clock.json (with the command), or None."""
    try:
        with open(os.path.join(ROOT, "profiles", "clock.json")) as f:
            return json.load(f)["workloads"][key]["clock_GHz"]
    except (OSError, KeyError, ValueError):
        return None


PEAK_CLOCK_GHZ = 2.4  # the engine clock MI355X's published dense f16 peak assumes


def decode_bytes(L, n_head, n_kv, hd):
    return 2 * L * n_kv * hd * 2 + 2 * n_head * hd * 2


def prefill_flops(M, p0, n_head, hd):
    return 4 * hd * n_head * (M * p0 + M * (M + 1) // 2)


class DecodeProblem:
    """Per-layer caches and the raw C-ABI launch of one decode attention call per layer."""

    def __init__(self, torch, gen, n_head, n_kv, hd, lens, layers, n_q=1, causal=False, shared=False, rope=None):
        from dooms_amd import _lib
        self.torch, self._lib = torch, _lib
        self.n_head, self.n_kv, self.hd, self.lens, self.layers, self.n_q = n_head, n_kv, hd, list(lens), layers, n_q
        self.rope = rope  # (mode, base): the fused step mx_attn_decode_rope on f32 q|k|v rows
        B = len(lens)
        dev = "cuda"
        if rope:
            self.q = torch.randn(B, (n_head + 2 * n_kv) * hd, generator=gen, device=dev)
            self.out = torch.empty(B, n_head * hd, dtype=torch.float32, device=dev)
        else:
            self.q = torch.randn(B * n_q, n_head * hd, generator=gen, device=dev).half()
            self.out = torch.empty(B * n_q, n_head * hd, dtype=torch.float16, device=dev)
        self.k, self.v = [], []
        for _ in range(layers):
            ks, vs = [], []
            for b, L in enumerate(lens):
                if shared and b > 0:
                    ks.append(ks[0]), vs.append(vs[0])
                    continue
                ks.append(torch.randn(L, n_kv * hd, generator=gen, device=dev).half())
                vs.append(torch.randn(L, n_kv * hd, generator=gen, device=dev).half())
            self.k.append(ks), self.v.append(vs)
        self.desc = _lib.make_desc(n_head, n_kv, hd, n_q, self.q.stride(0), n_kv * hd, n_head * hd,
                                   1.0 / math.sqrt(hd), causal=1 if causal else 0)
        need = _lib.decode_workspace_bytes(self.desc, B, max(lens))
        self.ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        _lib.check(_lib.decode_workspace_init(self.ws.data_ptr(), self.ws.numel(),
                                              torch.cuda.current_stream().cuda_stream))
        self.kp = [[t.data_ptr() for t in ks] for ks in self.k]
        self.vp = [[t.data_ptr() for t in vs] for vs in self.v]
        self.unique_bytes = sum(t.numel() * 2 for ks in self.k for t in set(ks)) * 2

    def launch(self, layer):
        _lib = self._lib
        if self.rope:
            _lib.check(_lib.decode_rope_raw(self.desc, self.rope[0], self.rope[1], self.lens, self.q.data_ptr(),
                                            self.kp[layer], self.vp[layer], self.out.data_ptr(), 0,
                                            self.ws.data_ptr(), self.ws.numel(),
                                            self.torch.cuda.current_stream().cuda_stream))
            return
        _lib.check(_lib.decode_raw(self.desc, self.lens, self.q.data_ptr(), self.kp[layer], self.vp[layer],
                                   self.out.data_ptr(), 0, self.ws.data_ptr(), self.ws.numel(),
                                   self.torch.cuda.current_stream().cuda_stream))

    def step(self):
        for l in range(self.layers):
            self.launch(l)

    def bytes_per_launch(self, shared=False):
        kv = sum(2 * L * self.n_kv * self.hd * 2 for L in (self.lens[:1] if shared else self.lens))
        return kv + len(self.lens) * self.n_q * 2 * self.n_head * self.hd * 2


class PrefillProblem:
    """Causal prompt chunks of `chunk` rows against the growing cache. workspace=True runs mx_attn_prefill_ws, the entry
    point the decoder's prompt path calls (the stream-K split over the CUs where planned); False mx_attn_prefill."""

    def __init__(self, torch, gen, n_head, n_kv, hd, N, chunk, layers=1, sigma=1.0, workspace=True, tuning=None):
        from dooms_amd import _lib
        self.torch, self._lib = torch, _lib
        self.n_head, self.n_kv, self.hd, self.N, self.chunk, self.layers = n_head, n_kv, hd, N, chunk, layers
        dev = "cuda"
        self.q = [(torch.randn(N, n_head * hd, generator=gen, device=dev) * sigma).half() for _ in range(layers)]
        self.k = [(torch.randn(N, n_kv * hd, generator=gen, device=dev) * sigma).half() for _ in range(layers)]
        self.v = [(torch.randn(N, n_kv * hd, generator=gen, device=dev) * sigma).half() for _ in range(layers)]
        self.out = torch.empty(N, n_head * hd, dtype=torch.float16, device=dev)
        self.chunks = [(p0, min(chunk, N - p0)) for p0 in range(0, N, chunk)]
        self.descs = [_lib.make_desc(n_head, n_kv, hd, M, n_head * hd, n_kv * hd, n_head * hd, 1.0 / math.sqrt(hd),
                                     p0=p0, causal=1, tuning=tuning) for p0, M in self.chunks]
        rs = n_head * hd * 2
        self.qoff = [p0 * rs for p0, _ in self.chunks]
        self.ws = None
        if workspace:
            nb = max(_lib.prefill_workspace_bytes(d) for d in self.descs)
            self.ws = torch.empty(max(nb, 256), dtype=torch.uint8, device=dev)
            _lib.check(_lib.decode_workspace_init(self.ws.data_ptr(), self.ws.numel(),
                                                  torch.cuda.current_stream().cuda_stream))

    def launch(self, layer, ci):
        _lib = self._lib
        p0, _ = self.chunks[ci]
        st = self.torch.cuda.current_stream().cuda_stream
        q, o = self.q[layer].data_ptr() + self.qoff[ci], self.out.data_ptr() + self.qoff[ci]
        if self.ws is None:
            _lib.check(_lib.prefill_raw(self.descs[ci], q, self.k[layer].data_ptr(), self.v[layer].data_ptr(), o, 0, st))
        else:
            _lib.check(_lib.prefill_ws_raw(self.descs[ci], q, self.k[layer].data_ptr(), self.v[layer].data_ptr(), o, 0,
                                           self.ws.data_ptr(), self.ws.numel(), st))

    def step(self):
        for l in range(self.layers):
            for ci in range(len(self.chunks)):
                self.launch(l, ci)

    def flops_per_layer(self):
        return sum(prefill_flops(M, p0, self.n_head, self.hd) for p0, M in self.chunks)


class LinearProblem:
    """mx_linear launches over `layers` distinct weight sets (so that weights stream from HBM), one input."""

    def __init__(self, torch, gen, M, N, K, flags, layers, count=1):
        from dooms_amd import _lib
        self.torch, self._lib = torch, _lib
        self.M, self.N, self.K, self.flags, self.layers, self.count = M, N, K, flags, layers, count
        dev = "cuda"
        self.x = torch.randn(M, K, generator=gen, device=dev)
        self.w = [[(torch.randn(N, K, generator=gen, device=dev) / math.sqrt(K)).half() for _ in range(count)]
                  for _ in range(layers)]
        out16 = bool(flags & _lib.LINEAR_OUT_F16)
        self.y = [torch.zeros(M, N, dtype=torch.float16 if out16 else torch.float32, device=dev) for _ in range(count)]
        self.gamma = torch.rand(K, generator=gen, device=dev) + 0.5
        self.bias = [torch.randn(N, generator=gen, device=dev) for _ in range(count)]
        self.desc = _lib.MxLinearDesc(M=M, N=N, K=K, flags=flags, x_stride=K, y_stride=N, eps=1e-5, reserved=0)
        nb = _lib.linear_workspace_bytes(self.desc)
        self.ws = torch.empty(max(nb, 256), dtype=torch.uint8, device=dev)
        self.nb = nb

    def step(self):
        _lib = self._lib
        stream = self.torch.cuda.current_stream().cuda_stream
        for l in range(self.layers):
            _lib.check(_lib.linear_raw(self.desc, [w.data_ptr() for w in self.w[l]], self.x.data_ptr(),
                                       [y.data_ptr() for y in self.y], self.gamma.data_ptr(),
                                       [b.data_ptr() for b in self.bias] if self.flags & _lib.LINEAR_BIAS else None,
                                       self.ws.data_ptr(), self.nb, self.torch.cuda.current_stream().cuda_stream))

    def weight_bytes(self):
        return 2 * self.N * self.K * self.count

    def flops(self):
        return 2 * self.M * self.N * self.K * self.count


class SelfAttentionProblem:
    """mx_self_attention (the IR SelfAttention op) on packed [B, N, 3E] rows."""

    def __init__(self, torch, gen, B, N, H, D, dtype):
        from dooms_amd import _lib
        self.torch, self._lib = torch, _lib
        codes = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}
        E = H * D
        self.B, self.N, self.E = B, N, E
        self.qkv = (torch.rand(B, N, 3 * E, generator=gen, device="cuda") * 2 - 1).to(dtype)
        self.y = torch.empty(B, N, E, dtype=dtype, device="cuda")
        self.desc = _lib.MxSelfAttnDesc(batch=B, n_tok=N, heads=H, embed=E, dtype=codes[dtype], scale=D ** -0.5)
        self.nb = _lib.self_attention_workspace_bytes(self.desc)
        self.ws = torch.empty(max(self.nb, 256), dtype=torch.uint8, device="cuda")

    def step(self):
        self._lib.check(self._lib.self_attention_raw(self.desc, self.qkv.data_ptr(), self.y.data_ptr(),
                                                     self.ws.data_ptr(), self.nb,
                                                     self.torch.cuda.current_stream().cuda_stream))

    def flops(self):
        return 4 * self.B * self.N * self.N * self.E  # the reference's cost model (src/ir/cost.cpp:30-34)


def cpu_info():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return model, avail


def cpu_decode_baseline(torch, prob, budget_s, threads):
    """The reference's CPU attention (oracle/oracle.c restatement) on the same decode workload, layer by layer until
    the time budget is spent. Returns (GB/s, layers timed, seconds)."""
    from oracle import oracle as O
    q = prob.q.float().cpu().numpy()
    hd, nh, nkv = prob.hd, prob.n_head, prob.n_kv
    host = []
    for l in range(min(prob.layers, 4)):  # the sample cycles over 4 layers' caches
        host.append([(prob.k[l][b].float().cpu().numpy(), prob.v[l][b].float().cpu().numpy()) for b in range(len(prob.lens))])
    done, t_total, nbytes = 0, 0.0, 0
    while t_total < budget_s or done == 0:
        kv = host[done % len(host)]
        t0 = time.perf_counter()
        for b, L in enumerate(prob.lens):
            O.cpu_attend_f32(q[b:b + 1], kv[b][0], kv[b][1], nh, nkv, hd, 1.0 / math.sqrt(hd), causal=False,
                             n_threads=threads)
        t_total += time.perf_counter() - t0
        nbytes += prob.bytes_per_launch()
        done += 1
    return nbytes / t_total / 1e9, done, t_total


def cpu_self_attention_baseline(sp, H, D, budget_s, threads):
    """The reference's CPU SelfAttention (attention_cpu_op, src/backend/ggml/ggml_backend.cpp:292-312: per (batch, head)
    scores, row softmax, weighted values in f32) through the restated CPU attention on the packed rows, timed per call."""
    from oracle import oracle as O
    x = sp.qkv.float().cpu().numpy()
    E = sp.E
    done, t = 0, 0.0
    while t < budget_s or done == 0:
        t0 = time.perf_counter()
        for b in range(sp.B):
            O.cpu_attend_f32(x[b, :, :E], x[b, :, E:2 * E], x[b, :, 2 * E:], H, H, D, D ** -0.5, causal=False,
                             n_threads=threads)
        t += time.perf_counter() - t0
        done += 1
    us = t / done * 1e6
    return {"us_per_call": round(us, 1), "TFLOPs": round(sp.flops() / (us * 1e-6) / 1e12, 4), "cores": threads,
            "kind": "port", "sample": f"{done} calls of the same shape through the restated CPU attention, {t:.1f} s"}


def cpu_gemv_baseline(lp, budget_s):
    """An f32 GEMV on the host (numpy's BLAS, all its threads) for the same weights: the reference's CPU matvec is
    llama.cpp/ggml, which is not buildable here, so this is a stand-in port, timed per launch."""
    import numpy as np
    w = lp.w[0][0].float().cpu().numpy()
    x = lp.x.cpu().numpy()
    done, t = 0, 0.0
    while t < budget_s or done == 0:
        t0 = time.perf_counter()
        _ = x @ w.T
        t += time.perf_counter() - t0
        done += 1
    us = t / done * 1e6
    return {"us_per_launch": round(us, 1), "GBps_weights_f32": round(4 * lp.N * lp.K / (us * 1e-6) / 1e9, 1),
            "kind": "port", "sample": f"{done} numpy f32 GEMVs (BLAS threads), {t:.1f} s"}


def cpu_prefill_baseline(torch, prob, budget_s, threads):
    """The restated CPU attention on sampled query rows of the prefill workload: rows taken from the end of the prompt
    (the most expensive ones) until the budget is spent; TFLOP/s over the unmasked pairs actually computed."""
    from oracle import oracle as O
    N, hd, nh, nkv = prob.N, prob.hd, prob.n_head, prob.n_kv
    k = prob.k[0].float().cpu().numpy()
    v = prob.v[0].float().cpu().numpy()
    q = prob.q[0].float().cpu().numpy()
    rows, t_total, flops = 0, 0.0, 0
    step = 8
    while t_total < budget_s or rows == 0:
        t1 = N - rows
        t0r = max(0, t1 - step)
        t0 = time.perf_counter()
        O.cpu_attend_f32(q[t0r:t1], k[:t1], v[:t1], nh, nkv, hd, 1.0 / math.sqrt(hd), p0=t0r, causal=True,
                         n_threads=threads)
        t_total += time.perf_counter() - t0
        flops += sum(4 * hd * nh * (t + 1) for t in range(t0r, t1))
        rows += t1 - t0r
        if t0r == 0:
            break
    return flops / t_total / 1e12, rows, t_total


def trace_decode(args):
    """Per-workgroup phase stamps of the decode kernel (the MX_ATTN_TRACE build), read after the graph-timed replays:
    the stamps are those of the last launch (the last layer of the last replay)."""
    import ctypes

    import numpy as np
    import torch
    from dooms_amd import _lib
    _lib.LIB_PATH = os.path.join(ROOT, "dooms_amd", "libmx_attn_trace.so")
    L = _lib.lib()
    L.mx_attn_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    L.mx_attn_trace_read.restype = ctypes.c_int
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    workloads = [("cfg3 Llama-3-8B batch 1, 8192 keys", 32, 8, 128, [8192], 1, 32),
                 ("cfg3 fused step (mx_attn_decode_rope), batch 1, 8192 keys", 32, 8, 128, [8192], 0, 32),
                 ("cfg1 Qwen2.5-0.5B, 513 keys", 14, 2, 64, [513], 1, 32),
                 ("cfg4 Whisper cross-attention, 1500 frames, greedy", 20, 20, 64, [1500], 1, 32),
                 ("cfg4 Whisper self-attention, 449 keys", 20, 20, 64, [449], 1, 32)]
    names = ["wave walk done", "waves merged", "partial published", "split counted", "splits merged",
             "merge: weights", "merge: accumulated"]
    for name, nh, nkv, hd, lens, nq, layers in workloads:
        # n_q 0 marks the fused step on the reference's f32 q|k|v rows (adjacent-pair rotary, base 500000)
        prob = DecodeProblem(torch, gen, nh, nkv, hd, lens, layers, n_q=max(nq, 1), rope=(0, 500000.0) if nq == 0 else None)
        ms, _ = time_graph(torch, prob.step, args.steps, args.warmup)
        buf = np.zeros(8192 * 16, dtype=np.uint64)
        assert L.mx_attn_trace_read(buf.ctypes.data, buf.nbytes) == 0
        t = buf.reshape(8192, 16).astype(np.int64)
        last = t[:, 0].max()
        t = t[t[:, 0] >= last - 5000]  # the last launch's workgroups (older stamps are > 50 us earlier)
        t0 = t[:, 0].min()
        rel = lambda col, sel: (col[sel] - t0) / 100.0  # the real-time clock ticks at 100 MHz
        # stamps older than the workgroup's own start are left from earlier launches (a workgroup of the grid's
        # padding returns after its start stamp)
        fresh = lambda col: np.where(col >= t[:, 0], col, 0)
        waves = np.where(t[:, 1:9] >= t[:, :1], t[:, 1:9], 0)
        walk = waves.max(axis=1)
        cols = [walk] + [fresh(t[:, c]) for c in (9, 10, 11, 12, 13, 15)]
        phases = {}
        for nm, col in zip(names, cols):
            sel = col > 0
            if sel.any():
                x = rel(col, sel)
                phases[nm] = {"p50": round(float(np.median(x)), 2), "max": round(float(x.max()), 2), "n": int(sel.sum())}
        print(json.dumps({"workload": name, "us_per_launch_graph": round(ms * 1000 / layers, 3),
                          "workgroups": int((walk > 0).sum()), "start_spread_us": round(float((t[:, 0].max() - t0) / 100), 2),
                          "phases_us_from_first_start": phases}), flush=True)
    return 0


def main():
    args = parse()
    if args.summarize:
        return summarize(args.summarize, args.kernel, args.last, args.per_dispatch)
    if args.trace_decode:
        return trace_decode(args)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the attention hot path has no multi-GPU path here "
                                   "(run with --gpus 1)", "n_gpus": args.gpus}))
        return 2
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    from dooms_amd import _lib
    _lib.lib()
    torch.backends.cuda.matmul.allow_tf32 = False
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    K, W = args.steps, args.warmup
    result = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": W, "higher_is_better": True,
              "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic"}
    extra = {}

    # same-run streaming copy (read + write), 1 GiB
    a = torch.empty(1 << 29, dtype=torch.float16, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    extra["copy_GBps"] = round(2 * a.numel() * 2 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    del a, b
    # same-run dense f16 GEMM through the vendor library (torch.matmul -> hipBLASLt), 8192^3: what the matrix cores
    # sustain on this box under its power limit, a second denominator beside the published 2.5 PFLOP/s
    a = torch.randn(8192, 8192, device="cuda", generator=gen).half()
    b = torch.randn(8192, 8192, device="cuda", generator=gen).half()
    for _ in range(3):
        c = a @ b.t()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(8):
        c = a @ b.t()
    e1.record()
    torch.cuda.synchronize()
    extra["f16_gemm_8192_TFLOPs"] = round(2 * 8192 ** 3 * 8 / (e0.elapsed_time(e1) * 1e-3) / 1e12, 1)
    del a, b, c

    model, ncpu = cpu_info()
    threads = max(1, min(16, ncpu))

    if args.only in ("decode", "all", "decode-headline"):
        # ---- headline: cfg3 decode, batch 1, L = 8192, 32 layers per step ----
        L = 8192
        dp = DecodeProblem(torch, gen, 32, 8, 128, [L], layers=32)
        ms, _ = time_graph(torch, dp.step, K, W)
        bpl = dp.bytes_per_launch()
        value = 32 * bpl / (ms * 1e-3) / 1e9
        avg_us = ms * 1e3 / 32  # one launch per layer, back to back in the graph
        achieved = bpl / (avg_us * 1e-6) / 1e9
        traffic = measured_traffic("decode_llama3_8b_b1_L8192")
        result.update({
            "value": round(value, 1), "ms_per_step": round(ms, 4),
            "config": {"workload": "cfg3 Llama-3-8B decode attention: 32 q / 8 kv heads, head_dim 128, batch 1, "
                                   "8192-token f16 KV cache, one query row; one step = 32 layers, each with its own "
                                   "K/V (1.07 GB per step)",
                       "batch": 1, "kv_len": L, "layers_per_step": 32, "n_head": 32, "n_head_kv": 8, "head_dim": 128,
                       "timing": "HIP graph replay of the 32-launch step, events on the launch stream"},
            "roofline": {"bound": "hbm", "kernel": "decode_kernel<128,4,false,8,true>", "achieved": round(achieved, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic, "bytes_per_launch": bpl, "avg_launch_us": round(avg_us, 3),
                         "launch_timing": "graph-timed region / launches (includes the gaps between launches)",
                         "copy_GBps": extra["copy_GBps"], "frac_of_copy": round(achieved / extra["copy_GBps"], 4),
                         "copy_note": "same-run 1 GiB device-to-device copy (read + write bytes / time)"},
        })
        if not args.no_cpu:
            v1, n1, t1 = cpu_decode_baseline(torch, dp, args.cpu_seconds, threads)
            v0, n0, t0 = cpu_decode_baseline(torch, dp, args.cpu_seconds / 4, 1)
            result["cpu_baseline"] = {
                "value": round(v1, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": f"{n1} layers of the same workload (batch 1, L=8192, 32/8 heads) through the restated "
                          f"CpuWhisperDecoder::attend (f32, double sum), {threads} threads over (row, head) tasks, "
                          f"{t1:.1f} s; host CPU: {model}, {ncpu} cores available",
                "single_thread_value": round(v0, 3), "single_thread_sample": f"{n0} layers, {t0:.1f} s"}
        del dp
        torch.cuda.empty_cache()

    if args.only in ("decode", "all"):
        # ---- cfg3 batched: lengths U[1024, 8192] by seed 3 ----
        # and batch 16 with every cache at 8192 keys (537 MB per launch: the rate the kernel sustains once the
        # launch and merge latency are amortized)
        rng = np.random.default_rng(3)
        for B, name in ((4, "decode_b4"), (16, "decode_b16"), (16, "decode_b16_L8192")):
            lens = [8192] * B if name.endswith("L8192") else [int(x) for x in rng.integers(1024, 8193, size=B)]
            layers = max(2, int(math.ceil(1.2e9 / (sum(lens) * 4096))))
            bp = DecodeProblem(torch, gen, 32, 8, 128, lens, layers=layers)
            ms_b, _ = time_graph(torch, bp.step, K, W)
            gbs = layers * bp.bytes_per_launch() / (ms_b * 1e-3) / 1e9
            extra[name] = {"GBps": round(gbs, 1), "us_per_layer": round(ms_b * 1e3 / layers, 2),
                           "roofline": {"bound": "hbm", "frac": round(gbs / HBM_PEAK_GBS, 4)},
                           "kv_lens": lens if len(set(lens)) > 1 else f"{B} x {lens[0]}", "layers_rotated": layers}
            del bp
            torch.cuda.empty_cache()

        # ---- the fused step (rotary embedding + cache append + attention), cfg3 batch 1, L = 8192, 32 layers ----
        fp = DecodeProblem(torch, gen, 32, 8, 128, [8192], layers=32, rope=(0, 500000.0))
        ms_f, _ = time_graph(torch, fp.step, K, W)
        extra["decode_rope_llama3_8b_b1_L8192"] = {
            "us_per_layer": round(ms_f * 1e3 / 32, 3),
            "GBps": round(32 * fp.bytes_per_launch() / (ms_f * 1e-3) / 1e9, 1),
            "roofline": {"bound": "hbm", "frac": round(32 * fp.bytes_per_launch() / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
            "note": "mx_attn_decode_rope: f32 q|k|v row in, q/k rotated, new k/v written at position 8191, f32 out"}
        del fp
        torch.cuda.empty_cache()

        # ---- cfg1 Qwen2.5-0.5B decode (513 keys, 24 layers) ----
        qp = DecodeProblem(torch, gen, 14, 2, 64, [513], layers=24)
        ms_q, _ = time_graph(torch, qp.step, K, W)
        extra["decode_qwen05b_513"] = {"us_per_layer": round(ms_q * 1e3 / 24, 3),
                                       "GBps": round(24 * qp.bytes_per_launch() / (ms_q * 1e-3) / 1e9, 1)}
        del qp
        # ---- cfg4 Whisper large-v3-turbo (4 decoder layers): self 448, cross 1500, batch 1 and beam 5 ----
        for beams in (1, 5):
            ws = DecodeProblem(torch, gen, 20, 20, 64, [448] * beams, layers=4)
            ms_s, _ = time_graph(torch, ws.step, K, W)
            wc = DecodeProblem(torch, gen, 20, 20, 64, [1500], layers=4, n_q=beams)
            ms_c, _ = time_graph(torch, wc.step, K, W)
            extra[f"whisper_beam{beams}"] = {
                "self_us_per_layer": round(ms_s * 1e3 / 4, 3),
                "self_GBps": round(4 * ws.bytes_per_launch() / (ms_s * 1e-3) / 1e9, 1),
                "cross_us_per_layer": round(ms_c * 1e3 / 4, 3),
                "cross_GBps": round(4 * wc.bytes_per_launch() / (ms_c * 1e-3) / 1e9, 1)}
            del ws, wc
        torch.cuda.empty_cache()

    if args.only in ("prefill", "all", "prefill-headline"):
        # ---- cfg5 Qwen2.5-7B 32k causal prefill in 2048-query chunks ----
        pp = PrefillProblem(torch, gen, 28, 4, 128, 32768, 2048, sigma=0.5)
        ms_p, _ = time_graph(torch, pp.step, K, W)
        fl = pp.flops_per_layer()
        tflops = fl / (ms_p * 1e-3) / 1e12
        avg_us = ms_p * 1e3 / len(pp.chunks)
        pre = {"metric": "prefill-attn TFLOP/s", "value": round(tflops, 1), "unit": "TFLOP/s",
               "ms_per_step": round(ms_p, 3),
               "workload": "cfg5 Qwen2.5-7B causal prefill: 28 q / 4 kv heads, head_dim 128, 32768 tokens in 16 "
                           "chunks of 2048 queries against the growing f16 cache, N(0, 0.5) inputs; FLOPs count "
                           "unmasked pairs only (7.697 TFLOP per step)",
               "flops_per_step": fl,
               "roofline": {"bound": "mfma", "kernel": "prefill_kernel<128,true,8,false,1,0> (chunks 1-15; chunk 0, the "
                                                        "whole first 2048 rows, on prefill_kernel<128,true,4,false,1,0>)",
                            "achieved": round(tflops, 1),
                            "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / F16_PEAK_TFLOPS, 4),
                            "traffic": measured_traffic("prefill_qwen7b_32k"), "avg_launch_us": round(avg_us, 2),
                            "launch_timing": "graph-timed region / launches; FLOPs per launch differ by chunk, so "
                                             "achieved = all FLOPs / all launch time"}}
        clk = measured_clock("prefill_qwen7b_32k")
        if clk:
            # the same peak at the shader clock the chip holds under this load (published peak x clock / 2.4 GHz)
            pk = F16_PEAK_TFLOPS * clk / PEAK_CLOCK_GHZ
            pre["roofline"].update({"clock_GHz": clk, "peak_at_clock": round(pk, 1),
                                    "frac_at_clock": round(tflops / pk, 4)})
        pre["roofline"]["same_run_gemm_TFLOPs"] = extra["f16_gemm_8192_TFLOPs"]
        pre["roofline"]["frac_of_same_run_gemm"] = round(tflops / extra["f16_gemm_8192_TFLOPs"], 4)
        if not args.no_cpu:
            v1, rows, t1 = cpu_prefill_baseline(torch, pp, args.cpu_seconds, threads)
            pre["cpu_baseline"] = {"value": round(v1, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
                                   "sample": f"the last {rows} query rows of the 32k prompt (all 28 heads, causal, "
                                             f"every visible key) through the restated CpuWhisperDecoder::attend, "
                                             f"{threads} threads, {t1:.1f} s; host CPU: {model}"}
        result["prefill"] = pre
        del pp
        torch.cuda.empty_cache()

    if args.only in ("prefill", "all"):
        # ---- cfg2 Qwen2.5-0.5B 512-token prompt: per layer and over 24 layers ----
        p2 = PrefillProblem(torch, gen, 14, 2, 64, 512, 512, layers=24)
        ms_2, _ = time_graph(torch, p2.step, K, W)
        fl2 = p2.flops_per_layer()
        extra["prefill_qwen05b_512"] = {
            "ms_24_layers": round(ms_2, 4), "us_per_layer": round(ms_2 * 1e3 / 24, 2),
            "TFLOPs": round(24 * fl2 / (ms_2 * 1e-3) / 1e12, 2),
            "reference_published_ms": 13.9,
            "reference_note": "M1 Pro GPU time of prompt attention for a 512-token prompt (site/data.js:142-146); "
                              "a different metric and machine, so vs_baseline stays null"}
        del p2
        # ---- the reference's prompt path on its f32 q|k|v rows (mx_attn_prefill_rope: rope_store + attention),
        # cfg5's 32k prompt in 2048-row chunks, split-half rotation (Qwen2), base 1e6 ----
        from dooms_amd import _lib as L
        nq, nkv, hd, N, C = 28, 4, 128, 32768, 2048
        qkv = torch.randn(N, (nq + 2 * nkv) * hd, generator=gen, device="cuda") * 0.5
        kc = torch.empty(N, nkv * hd, dtype=torch.float16, device="cuda")
        vc = torch.empty_like(kc)
        o32 = torch.empty(N, nq * hd, dtype=torch.float32, device="cuda")
        rdescs = [L.make_desc(nq, nkv, hd, C, qkv.stride(0), kc.stride(0), o32.stride(0), 1.0 / math.sqrt(hd),
                              p0=p0, causal=1) for p0 in range(0, N, C)]

        def rope_step():
            for ci, d in enumerate(rdescs):
                p0 = ci * C
                L.check(L.prefill_rope_raw(d, 1, 1e6, qkv.data_ptr() + p0 * qkv.stride(0) * 4, kc.data_ptr(),
                                           vc.data_ptr(), o32.data_ptr() + p0 * o32.stride(0) * 4, 0,
                                           torch.cuda.current_stream().cuda_stream))
        ms_r, _ = time_graph(torch, rope_step, max(3, K // 4), max(1, W // 2))
        fl_r = sum(prefill_flops(C, p0, nq, hd) for p0 in range(0, N, C))
        tf_r = fl_r / (ms_r * 1e-3) / 1e12
        extra["prefill_rope_qwen7b_32k"] = {
            "ms_per_step": round(ms_r, 3), "TFLOPs": round(tf_r, 1),
            "roofline": {"bound": "mfma", "frac": round(tf_r / F16_PEAK_TFLOPS, 4)},
            "note": "mx_attn_prefill_rope per 2048-row chunk: f32 q|k|v rows in, keys/values rotated into the f16 "
                    "caches (rope_store_kernel), queries rotated in the attention kernel, f32 out; same FLOPs as the "
                    "prefill line"}
        del qkv, kc, vc, o32
        torch.cuda.empty_cache()

    if args.only in ("linear", "all"):
        # ---- the projections either side of the attention (mx_linear): Llama-3-8B shapes, Whisper cross cache ----
        from dooms_amd import _lib as L
        lin = {}
        # kernel: this library's kernels that produced the figure (mx_linear loads no vendor GEMM library)
        for name, M, N, Kd, flags, layers, count, kernel in [
                ("gemv_qkv_llama3_8b", 1, 6144, 4096, L.LINEAR_RMS_NORM, 32, 1, "gemv_kernel"),
                ("gemv_attn_output_llama3_8b", 1, 4096, 4096, L.LINEAR_ACCUMULATE, 32, 1, "gemv_kernel"),
                ("gemm_qkv_llama3_8b_chunk2048", 2048, 6144, 4096, L.LINEAR_RMS_NORM, 4, 1,
                 "stage_kernel + gemm_w192_kernel"),
                ("whisper_cross_kv_1500x1280_4layers", 1500, 1280, 1280, L.LINEAR_OUT_F16 | L.LINEAR_BIAS, 1, 8,
                 "stage_kernel + gemm_big_kernel")]:
            lp = LinearProblem(torch, gen, M, N, Kd, flags, layers, count)
            ms_l, _ = time_graph(torch, lp.step, max(5, K), max(1, W))
            us = ms_l * 1e3 / layers
            e = {"M": M, "N": N, "K": Kd, "count": count, "kernel": kernel, "us_per_launch": round(us, 2)}
            if M <= 8:
                e["GBps_weights"] = round(lp.weight_bytes() / (us * 1e-6) / 1e9, 1)
                e["roofline"] = {"bound": "hbm", "frac": round(e["GBps_weights"] / HBM_PEAK_GBS, 4)}
            else:
                e["TFLOPs"] = round(lp.flops() / (us * 1e-6) / 1e12, 1)
                e["roofline"] = {"bound": "mfma", "frac": round(e["TFLOPs"] / F16_PEAK_TFLOPS, 4)}
            if not args.no_cpu and M == 1 and name.startswith("gemv_qkv"):
                e["cpu_baseline"] = cpu_gemv_baseline(lp, min(5.0, args.cpu_seconds))
            lin[name] = e
            del lp
            torch.cuda.empty_cache()
        # the vendor GEMM on the same chunk shape for comparison only (torch.matmul -> hipBLASLt, f16 in and out, no
        # norm or staging): not part of this library
        xa = torch.randn(2048, 4096, generator=gen, device="cuda").half()
        wv = [torch.randn(6144, 4096, generator=gen, device="cuda").half() for _ in range(4)]
        yv = torch.empty(2048, 6144, dtype=torch.float16, device="cuda")

        def vendor_step():
            for w_ in wv:
                torch.matmul(xa, w_.t(), out=yv)
        ms_v, _ = time_graph(torch, vendor_step, max(5, K), max(1, W))
        us_v = ms_v * 1e3 / len(wv)
        lin["vendor_torch_matmul_qkv_chunk2048"] = {
            "M": 2048, "N": 6144, "K": 4096, "us_per_launch": round(us_v, 2),
            "TFLOPs": round(2 * 2048 * 6144 * 4096 / (us_v * 1e-6) / 1e12, 1),
            "note": "torch.matmul (hipBLASLt) on f16 operands of the same shape, for comparison; not this library"}
        del xa, wv, yv
        extra["linear"] = lin

    if args.only in ("self-attention", "all"):
        # ---- the IR SelfAttention op (mx_self_attention): ViT shapes ----
        sa = {}
        for name, B, N, H, D, dt in [("vit_h_210x16x80_f32", 1, 210, 16, 80, torch.float32),
                                     ("vit_b16_384px_b8_f16", 8, 577, 12, 64, torch.float16),
                                     ("vit_l_1024tok_b4_bf16", 4, 1024, 16, 64, torch.bfloat16)]:
            sp = SelfAttentionProblem(torch, gen, B, N, H, D, dt)
            reps = 16

            def step(sp=sp):
                for _ in range(reps):
                    sp.step()
            ms_s, _ = time_graph(torch, step, max(5, K), max(1, W))
            us = ms_s * 1e3 / reps
            tf = sp.flops() / (us * 1e-6) / 1e12
            sa[name] = {"us_per_call": round(us, 2), "TFLOPs": round(tf, 2), "flops_per_call": sp.flops(),
                        "roofline": {"bound": "mfma", "frac": round(tf / F16_PEAK_TFLOPS, 4)}}
            if not args.no_cpu and name.startswith("vit_h"):
                sa[name]["cpu_baseline"] = cpu_self_attention_baseline(sp, H, D, min(5.0, args.cpu_seconds), threads)
            del sp
        extra["self_attention"] = sa

    if "value" not in result and "prefill" not in result:  # --only linear / self-attention: their first figure
        if "linear" in extra:
            e = extra["linear"]["gemv_qkv_llama3_8b"]
            result.update({"value": e["GBps_weights"], "unit": "GB/s",
                           "config": {"workload": "mx_linear q|k|v GEMV, Llama-3-8B (M 1, N 6144, K 4096)"}})
        else:
            e = extra["self_attention"]["vit_b16_384px_b8_f16"]
            result.update({"value": e["TFLOPs"], "unit": "TFLOP/s",
                           "config": {"workload": "mx_self_attention, ViT-B/16 384 px, batch 8 (577 tokens, 12 x 64)"}})
    if "value" not in result:  # --only prefill*: the prefill figure is the line's value
        pre = result["prefill"]
        result.update({"value": pre["value"], "unit": pre["unit"], "ms_per_step": pre["ms_per_step"],
                       "config": {"workload": pre["workload"]}, "roofline": pre["roofline"]})
        if "cpu_baseline" in pre:
            result["cpu_baseline"] = pre["cpu_baseline"]
    result["extra"] = extra
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

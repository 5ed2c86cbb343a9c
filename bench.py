#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-GEMM path (one GPU).

Headline metric: "W4A16 decode GB/s (% HBM peak) + W8A8
prefill TOPS (% MFMA peak), 1 GPU".

* ``value`` -- W4A16 decode GEMV, M=1, K=8192, N=28672, asymmetric int4
  group 128 (fp16 scales, u4 zero points), bf16 activations and output: the
  north-star shape.  One step = one GEMM launch over one weight matrix; the
  launches rotate over enough distinct weight sets (> 2x the 256 MB Infinity
  Cache) that every step streams its weights from HBM.  Throughput is the
  algorithmic bytes of one call (packed weights + scales + zeros + activations
  + output) times K steps over the timed region.
* ``w8a8_prefill`` -- int8 x int8 -> int32 -> fp32 scale -> bf16, M=4096,
  K=4096, N=14336 (north-star target) and M=2048 (config 3): TOPS = 2*M*K*N
  per call over the measured launch time.
* ``roofline`` -- the W4A16 decode kernel against the 8 TB/s HBM peak, with
  HBM traffic per launch from the committed rocprofv3 PMC summary.
* ``cpu_baseline`` -- the reference's own gemm_w4a16_groupwise
  (gemm_quant.cpp:54-82, compiled from its sources into oracle/_ref) or, where
  that library is absent, the C restatement in oracle/, timed on the host on
  the same M=1, K=8192, N=28672 shape (fp32 API, symmetric int4 -- the only
  form the reference has), single thread as the reference runs.

Timing: launches are captured into HIP graphs (torch.cuda.CUDAGraph drives
hipStreamBeginCapture on the stream the kernels are launched on) so the
timed region measures the GPU, not Python; HIP events bracket the region on
that same stream, opened behind a short spin kernel so that the host's
submission of the graphs is not inside it.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA, published
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA, published
FP8_PEAK_TFLOPS = 5000.0    # MI355X dense fp8 MFMA, published
INFINITY_CACHE_BYTES = 256 << 20


def w4a16_bytes(M: int, K: int, N: int, G: int) -> int:
    """Algorithmic bytes of one asymmetric W4A16 call (u4 weights, fp16
    scales, u4 zeros, bf16 activations and output)."""
    return K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2 + M * K * 2 + M * N * 2


def w4a16_sym_f32_bytes(M: int, K: int, N: int, G: int) -> int:
    """Algorithmic bytes of the reference's fp32-API call (int4 weights, fp32
    scales, fp32 activations and output)."""
    return K * N // 2 + (K // G) * N * 4 + M * K * 4 + M * N * 4


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# GPU legs
# ---------------------------------------------------------------------------

class GraphTimer:
    """Times exactly `steps` launches of `launch(i)`, captured in HIP graphs
    of `chunk` launches (direct=False) or launched straight onto the stream
    (direct=True: for launches long enough that the host, enqueueing while a
    spin kernel runs, stays ahead of the GPU; a graph replay adds a startup
    cost of several microseconds on the GPU, which a short run amortizes
    over few launches)."""

    def __init__(self, launch, period: int, chunk: int, direct: bool = False):
        import torch
        self.torch = torch
        self.launch = launch
        self.period = period
        self.chunk = max(1, chunk)
        self.direct = direct
        self._graphs = {}
        self.host_enqueue_ms = None

    def _graph(self, n: int, start: int):
        key = (n, start % self.period)
        g = self._graphs.get(key)
        if g is None:
            torch = self.torch
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    for i in range(n):
                        self.launch(start + i)
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            self._graphs[key] = g
        return g

    def run(self, steps: int) -> None:
        if self.direct:
            for i in range(steps):
                self.launch(i)
            return
        done = 0
        while done < steps:
            n = min(self.chunk, steps - done)
            self._graph(n, done).replay()
            done += n

    def prepare(self, steps: int) -> None:
        if self.direct:
            return
        done = 0
        while done < steps:
            n = min(self.chunk, steps - done)
            self._graph(n, done)
            done += n

    def time(self, steps: int, warmup: int):
        """Returns (elapsed ms of the timed region by HIP events, wall ms).
        Order on the stream: a spin kernel (~1 ms; the host enqueues the
        rest while it runs), the `warmup` untimed launches, the opening
        event, exactly `steps` launches, the closing event.  The warm-up
        launches run immediately before the timed ones, so the timed region
        starts with clocks, caches and TLBs as the steady state has them,
        and the events bracket the GPU's execution of the steps, not the
        host's launch latency."""
        torch = self.torch
        self.prepare(steps)
        if warmup:
            self.prepare(warmup)
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        torch.cuda._sleep(2_000_000)
        if warmup:
            self.run(warmup)
        ev0.record()
        h0 = time.perf_counter()
        self.run(steps)
        self.host_enqueue_ms = (time.perf_counter() - h0) * 1e3
        ev1.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3
        return ev0.elapsed_time(ev1), wall

    def chunk_percentiles(self, steps: int, min_chunks: int = 10):
        """A second pass with a HIP event after every graph replay (a chunk
        of back-to-back launches), over max(steps, min_chunks * chunk)
        launches so that the percentiles rest on at least `min_chunks`
        chunks whatever `steps` is: returns the 50th and 90th percentiles
        over the chunks of the time per launch, in us.  Run apart from
        time() so its events do not enter the reported total."""
        torch = self.torch
        steps = max(steps, min_chunks * self.chunk)
        self.prepare(steps)
        torch.cuda.synchronize()
        torch.cuda._sleep(2_000_000)
        self.run(self.chunk)  # one untimed chunk: the first timed one does not start cold
        evs = [torch.cuda.Event(enable_timing=True)]
        evs[0].record()
        sizes = []
        done = 0
        while done < steps:
            n = min(self.chunk, steps - done)
            if self.direct:
                for i in range(done, done + n):
                    self.launch(i)
            else:
                self._graph(n, done).replay()
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            evs.append(e)
            sizes.append(n)
            done += n
        torch.cuda.synchronize()
        per = sorted(evs[i].elapsed_time(evs[i + 1]) * 1e3 / sizes[i] for i in range(len(sizes)))
        def pct(q):
            return per[min(len(per) - 1, int(round(q * (len(per) - 1))))]
        return pct(0.5), pct(0.9)


def make_w4_sets(ops, K: int, N: int, G: int, nsets: int, seed: int):
    """`nsets` distinct asymmetric int4 weight sets quantized on the device
    from N(0, 0.02), prepacked; plus bf16 N(0,1) activation rows."""
    import numpy as np
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    sets = []
    for _ in range(nsets):
        W = torch.randn((K, N), generator=gen, device="cuda", dtype=torch.float32) * 0.02
        packed = ops.empty((K // 2, N), np.uint8)
        sc = ops.empty((K // G, N), np.uint16)
        zp = ops.empty((K // G, N), np.uint8)
        ops.lib().call("lhq_q4a_quantize_groupwise", W.data_ptr(), packed.data_ptr(), sc.data_ptr(),
                       zp.data_ptr(), K, N, G, ops.stream())
        del W
        sets.append(ops.prepack_w4_asym(packed, sc, zp, K, N, G))
        del packed, sc, zp
    torch.cuda.synchronize()
    return sets


def bench_w4a16_f32(ops, M, K, N, G, steps, warmup, seed=0, min_rotate_bytes=2 * INFINITY_CACHE_BYTES + (1 << 26),
                    workspace=False):
    """The reference interface (lhq_gemm_w4a16, gemm_quant.cpp:54-82): fp32
    activations and output, symmetric int4 weights with fp32 group scales,
    alpha = 1, beta = 0; timed over rotating weight sets like the bf16 legs.
    workspace: through lhq_gemm_w4a16_ws with the workspace the shape asks
    for (K split across workgroups at thin grids; the lh:: drop-in's route).
    Bytes: K*N/2 codes + (K/G)*N*4 scales + M*K*4 + M*N*4."""
    import numpy as np
    import torch
    per = K * N // 2 + (K // G) * N * 4 + M * K * 4 + M * N * 4
    nsets = max(2, -(-min_rotate_bytes // per))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    sets = []
    for _ in range(nsets):
        packed = torch.randint(0, 256, (K // 2, N), dtype=torch.uint8, device="cuda", generator=gen)
        sc = torch.rand((K // G, N), device="cuda", generator=gen) * 0.01
        sets.append(ops.prepack_w4_sym(packed, sc, K, N, G))
        del packed, sc
    A = [torch.randn((M, K), generator=gen, device="cuda") for _ in range(nsets)]
    C = [torch.zeros((M, N), device="cuda") for _ in range(nsets)]
    L = ops.lib().cdll
    ws_bytes = L.lhq_gemm_w4a16_workspace_bytes(M, N, K, G) if workspace else 0
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")

    def launch(i):
        j = i % nsets
        if workspace:
            st = L.lhq_gemm_w4a16_ws(A[j].data_ptr(), sets[j].qweight.data_ptr(), sets[j].scales.data_ptr(),
                                     C[j].data_ptr(), M, N, K, G, 1.0, 0.0, ws.data_ptr(), ws_bytes, ops.stream())
        else:
            st = L.lhq_gemm_w4a16(A[j].data_ptr(), sets[j].qweight.data_ptr(), sets[j].scales.data_ptr(),
                                  C[j].data_ptr(), M, N, K, G, 1.0, 0.0, ops.stream())
        if st:
            raise RuntimeError(f"lhq_gemm_w4a16: {ops.lib().last_error()}")

    timer = GraphTimer(launch, nsets, chunk=nsets * max(1, 64 // nsets))
    ms, _ = timer.time(steps, warmup)
    us = ms * 1e3 / steps
    res = {"leg": "w4a16_f32_interface", "M": M, "K": K, "N": N, "G": G,
           "entry": "lhq_gemm_w4a16_ws" if workspace else "lhq_gemm_w4a16", "workspace_bytes": ws_bytes,
           "us_per_call": round(us, 2), "gbs": round(per / (us * 1e-6) / 1e9, 1),
           "hbm_frac": round(per / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
           "tflops": round(2.0 * M * K * N / (us * 1e-6) / 1e12, 1),
           "mfma_frac": round(2.0 * M * K * N / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)}
    del timer, sets, A, C, ws
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def bench_w4a16(ops, M, K, N, G, steps, warmup, seed=0, min_rotate_bytes=2 * INFINITY_CACHE_BYTES + (1 << 26),
                workspace=False, direct=False):
    """W4A16 bf16 timed over rotating weight sets.  workspace: through
    lhq_gemm_w4a16_bf16_ws with the workspace the shape asks for (K split
    across workgroups where the grid is thin), else lhq_gemm_w4a16_bf16.
    direct: launches straight onto the stream instead of graph replays."""
    import numpy as np
    import torch
    per = w4a16_bytes(M, K, N, G)
    nsets = max(2, -(-min_rotate_bytes // per))
    sets = make_w4_sets(ops, K, N, G, nsets, seed)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 1)
    A = [(torch.randn((M, K), generator=gen, device="cuda") .to(torch.bfloat16)).view(torch.int16)
         for _ in range(nsets)]
    C = [ops.empty((M, N), np.int16) for _ in range(nsets)]
    args = [(A[i].data_ptr(), sets[i].qweight.data_ptr(), sets[i].scales.data_ptr(),
             sets[i].zeros.data_ptr(), C[i].data_ptr()) for i in range(nsets)]
    ws_bytes = ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, G) if workspace else 0
    ws = ops.empty((max(ws_bytes, 1),), np.uint8)
    name = "lhq_gemm_w4a16_bf16_ws" if workspace else "lhq_gemm_w4a16_bf16"
    fn = getattr(ops.lib().cdll, name)
    extra = (ws.data_ptr(), ws_bytes) if workspace else ()

    def launch(i):
        a = args[i % nsets]
        st = fn(a[0], a[1], a[2], a[3], a[4], M, N, K, G, *extra, ops.stream())
        if st:
            raise RuntimeError(f"{name}: {ops.lib().last_error()}")

    timer = GraphTimer(launch, nsets, chunk=nsets * max(1, 64 // nsets), direct=direct)
    ms, wall = timer.time(steps, warmup)
    us = ms * 1e3 / steps
    host_ms = timer.host_enqueue_ms
    p50, p90 = timer.chunk_percentiles(steps)
    res = {"M": M, "K": K, "N": N, "G": G, "entry": name, "workspace_bytes": ws_bytes,
           "bytes_per_call": per, "weight_sets": nsets,
           "rotate_bytes": per * nsets, "us_per_call": us, "gbs": per / (us * 1e-6) / 1e9,
           "elapsed_ms": ms, "wall_ms": wall, "chunk_launches": timer.chunk,
           "launch": "direct" if direct else "graph", "host_enqueue_ms": host_ms,
           "us_p50_chunk": p50, "us_p90_chunk": p90}
    res["hbm_frac"] = res["gbs"] / HBM_PEAK_GBS
    del timer, sets, A, C, ws
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def bench_moe(ops, steps, warmup, seed=0, T=512, E=8, topk=2, K=4096, N=14336, G=128):
    """Config 4: ragged grouped W4A16 over E experts in one launch.  T tokens
    each pick `topk` distinct experts (top-k of seeded uniform scores); the
    dispatched rows are expert-major and the group table is the exclusive
    prefix sum of the per-expert counts (moe.cpp:111-123)."""
    import numpy as np
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    scores = torch.rand((T, E), generator=gen, device="cuda")
    ids = torch.topk(scores, topk, dim=1).indices.flatten()
    counts = torch.bincount(ids, minlength=E).cpu().numpy()
    off = np.zeros(E + 1, np.int32)
    off[1:] = np.cumsum(counts)
    rows = int(off[-1])
    sets = make_w4_sets(ops, K, N, G, E, seed)
    A = torch.randn((rows, K), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    C = ops.empty((rows, N), np.int16)
    offd = torch.tensor(off, device="cuda")
    qptr = torch.tensor([w.qweight.data_ptr() for w in sets], dtype=torch.int64, device="cuda")
    sptr = torch.tensor([w.scales.data_ptr() for w in sets], dtype=torch.int64, device="cuda")
    zptr = torch.tensor([w.zeros.data_ptr() for w in sets], dtype=torch.int64, device="cuda")
    L = ops.lib().cdll
    # the persistent launch (its workspace, as the query sizes it) and the
    # one-workgroup-per-tile grid without one
    ws_bytes = L.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(E, rows, N, K, G)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")

    def launcher(persistent):
        def launch(_i):
            if persistent:
                st = L.lhq_gemm_w4a16_bf16_grouped_ws(A.data_ptr(), offd.data_ptr(), qptr.data_ptr(), sptr.data_ptr(),
                                                      zptr.data_ptr(), C.data_ptr(), E, rows, N, K, G, ws.data_ptr(),
                                                      ws_bytes, ops.stream())
            else:
                st = L.lhq_gemm_w4a16_bf16_grouped(A.data_ptr(), offd.data_ptr(), qptr.data_ptr(), sptr.data_ptr(),
                                                   zptr.data_ptr(), C.data_ptr(), E, rows, N, K, G, ops.stream())
            if st:
                raise RuntimeError(f"grouped W4A16: {ops.lib().last_error()}")
        return launch

    ms_grid, _ = GraphTimer(launcher(False), 1, chunk=16).time(steps, warmup)
    ms, _ = GraphTimer(launcher(True), 1, chunk=16).time(steps, warmup)
    us = ms * 1e3 / steps
    flops = 2 * rows * K * N
    byts = E * (K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2) + rows * K * 2 + rows * N * 2
    res = {"tokens": T, "experts": E, "top_k": topk, "rows": rows, "rows_per_expert": counts.tolist(),
           "K": K, "N": N, "G": G, "us_per_call": us, "tflops": flops / (us * 1e-6) / 1e12,
           "gbs": byts / (us * 1e-6) / 1e9, "flops": flops, "bytes": byts,
           "launch": "persistent tile scheduler (lhq_gemm_w4a16_bf16_grouped_ws; split along K below one round)",
           "workspace_bytes": ws_bytes, "us_per_call_grid": ms_grid * 1e3 / steps}
    res["mfma_frac"] = res["tflops"] / BF16_PEAK_TFLOPS
    res["hbm_frac"] = res["gbs"] / HBM_PEAK_GBS
    del sets, A, C, ws
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def bench_fp8(ops, M, K, N, steps, warmup, seed=0):
    """gemm_fp8_e4m3 (gemm_quant.cpp:87-104): e4m3 A [M,K] and B [K,N] quantized
    per tensor on the device from N(0,1) / N(0,0.02), fp32 C = sA*sB*acc."""
    import numpy as np
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    L = ops.lib()
    W = torch.randn((K, N), generator=gen, device="cuda") * 0.02
    B8 = ops.empty((K, N), np.uint8)
    sB = ops.empty((1,), np.float32)
    L.call("lhq_fp8_quantize_per_tensor", W.data_ptr(), B8.data_ptr(), sB.data_ptr(), K * N, ops.stream())
    del W
    Bt = ops.prepack_b8(B8, K, N)
    del B8
    X = torch.randn((M, K), generator=gen, device="cuda")
    A8 = ops.empty((M, K), np.uint8)
    sA = ops.empty((1,), np.float32)
    L.call("lhq_fp8_quantize_per_tensor", X.data_ptr(), A8.data_ptr(), sA.data_ptr(), M * K, ops.stream())
    del X
    C = ops.empty((M, N), np.float32)
    fn = L.cdll.lhq_gemm_fp8_e4m3

    def launch(_i):
        st = fn(A8.data_ptr(), Bt.data_ptr(), sA.data_ptr(), sB.data_ptr(), C.data_ptr(), M, N, K, 1.0, 0.0,
                ops.stream())
        if st:
            raise RuntimeError(f"lhq_gemm_fp8_e4m3: {L.last_error()}")

    ms, _ = GraphTimer(launch, 1, chunk=16).time(steps, warmup)
    us = ms * 1e3 / steps
    tf = 2 * M * K * N / (us * 1e-6) / 1e12
    # the register-only MFMA rate on these same e4m3 values, and the same
    # GEMM on all-zero operands (which hold a higher clock)
    same = operand_probe(ops, 1, A8, Bt, iters=2000)
    Az = torch.zeros_like(A8)
    Bz = torch.zeros_like(Bt)

    def zlaunch(_i):
        st = fn(Az.data_ptr(), Bz.data_ptr(), sA.data_ptr(), sB.data_ptr(), C.data_ptr(), M, N, K, 1.0, 0.0,
                ops.stream())
        if st:
            raise RuntimeError(f"lhq_gemm_fp8_e4m3: {L.last_error()}")

    zms, _ = GraphTimer(zlaunch, 1, chunk=16).time(steps, warmup)
    zus = zms * 1e3 / steps
    del Bt, A8, C, Az, Bz
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"leg": "fp8_e4m3_gemm", "M": M, "K": K, "N": N, "us_per_call": round(us, 2), "tflops": round(tf, 1),
            "peak": FP8_PEAK_TFLOPS, "mfma_frac": round(tf / FP8_PEAK_TFLOPS, 4),
            "sustained_same_operands": same, "frac_of_sustained": round(tf / same["value"], 4),
            "us_zero_operands": round(zus, 2)}


def bench_moe_layer(ops, steps, warmup, seed=0, T=512, E=8, topk=2, H=4096, I=14336, G=128):
    """Config 4's MoE layer end to end on the device (moe.cpp:102-221 with
    W4A16 experts): dispatch -> gate/up projection with the SwiGLU epilogue
    -> down projection -> combine, Mixtral shapes.  Each stage is timed on its
    own (HIP graphs of `steps` launches), then the chain."""
    import numpy as np
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    scores = torch.rand((T, E), generator=gen, device="cuda")
    top = torch.topk(scores, topk, dim=1)
    ids = top.indices.to(torch.int32).contiguous()
    gates = torch.softmax(top.values, dim=1).contiguous()
    S = T * topk
    x = torch.randn((T, H), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    gate = make_w4_sets(ops, H, I, G, E, seed + 1)
    up = make_w4_sets(ops, H, I, G, E, seed + 2)
    gu = [ops.interleave_gate_up(a, b) for a, b in zip(gate, up)]
    del gate, up
    down = make_w4_sets(ops, I, H, G, E, seed + 3)
    guq, gus, guz = ops.pointer_tables(gu)
    dq, ds, dz = ops.pointer_tables(down)
    off = ops.zeros((E + 1,), np.int32)
    tok, slot, pos = (ops.zeros((S,), np.int32) for _ in range(3))
    xs = ops.empty((S, H), np.int16)
    act = ops.empty((S, I), np.int16)
    y = ops.empty((S, H), np.int16)
    out = ops.empty((T, H), np.int16)
    L = ops.lib()
    st = ops.stream
    # one workspace for both grouped launches (they run in order on the stream)
    ws_bytes = max(L.cdll.lhq_gemm_w4a16_bf16_grouped_swiglu_workspace_bytes(E, S, I, H, G),
                   L.cdll.lhq_gemm_w4a16_bf16_grouped_workspace_bytes(E, S, H, I, G))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")

    def chk(name, status):
        if status:
            raise RuntimeError(f"{name}: {L.last_error()}")

    def dispatch(_i):
        chk("dispatch", L.cdll.lhq_moe_dispatch_bf16(x.data_ptr(), ids.data_ptr(), off.data_ptr(), tok.data_ptr(),
                                                     slot.data_ptr(), pos.data_ptr(), xs.data_ptr(), T, H, E, topk,
                                                     st()))

    def gate_up(_i):
        chk("gate_up", L.cdll.lhq_gemm_w4a16_bf16_grouped_swiglu_ws(xs.data_ptr(), off.data_ptr(), guq.data_ptr(),
                                                                    gus.data_ptr(), guz.data_ptr(), act.data_ptr(), E,
                                                                    S, I, H, G, ws.data_ptr(), ws_bytes, st()))

    def down_proj(_i):
        chk("down", L.cdll.lhq_gemm_w4a16_bf16_grouped_ws(act.data_ptr(), off.data_ptr(), dq.data_ptr(), ds.data_ptr(),
                                                          dz.data_ptr(), y.data_ptr(), E, S, H, I, G, ws.data_ptr(),
                                                          ws_bytes, st()))

    def combine(_i):
        chk("combine", L.cdll.lhq_moe_combine_bf16(y.data_ptr(), pos.data_ptr(), gates.data_ptr(), out.data_ptr(),
                                                   T, H, topk, st()))

    def layer(i):
        dispatch(i)
        gate_up(i)
        down_proj(i)
        combine(i)

    dispatch(0)
    torch.cuda.synchronize()
    rows = (off[1:] - off[:-1]).cpu().numpy().tolist()
    # weights of the experts that hold rows (the kernels read no others)
    active = sum(1 for r in rows if r > 0)
    wbytes = lambda K, N: active * (K * N // 2 + (K // G) * N * 2 + (K // G) * N // 2)  # noqa: E731
    stages = {
        "dispatch": (dispatch, 0, T * H * 2 + S * H * 2 + T * topk * 4 * 4),
        "gate_up_swiglu": (gate_up, 2 * S * H * 2 * I, wbytes(H, 2 * I) + S * H * 2 + S * I * 2),
        "down": (down_proj, 2 * S * I * H, wbytes(I, H) + S * I * 2 + S * H * 2),
        "combine": (combine, 0, S * H * 2 + T * H * 2 + T * topk * 8),
    }
    res = {"tokens": T, "experts": E, "top_k": topk, "hidden": H, "intermediate": I, "G": G,
           "rows_per_expert": rows, "grouped_launches": "persistent (the _ws entry points)",
           "workspace_bytes": ws_bytes, "stages": {}}
    total_flops = total_bytes = 0
    for name, (fn, flops, byts) in stages.items():
        n = steps if flops else 4 * steps
        ms, _ = GraphTimer(fn, 1, chunk=16).time(n, max(2, warmup))
        us = ms * 1e3 / n
        r = {"us": round(us, 2), "gbs": round(byts / (us * 1e-6) / 1e9, 1),
             "hbm_frac": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes": byts}
        if flops:
            tf = flops / (us * 1e-6) / 1e12
            r.update({"tflops": round(tf, 1), "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4), "flops": flops})
        res["stages"][name] = r
        total_flops += flops
        total_bytes += byts
    ms, _ = GraphTimer(layer, 1, chunk=8).time(steps, max(2, warmup))
    us = ms * 1e3 / steps
    res.update({"layer_us": round(us, 2), "tokens_per_s": round(T / (us * 1e-6), 1),
                "layer_tflops": round(total_flops / (us * 1e-6) / 1e12, 1),
                "layer_gbs": round(total_bytes / (us * 1e-6) / 1e9, 1)})
    del gu, down, x, xs, act, y, out, ws
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def bench_w8a8(ops, M, K, N, steps, warmup, seed=0):
    import numpy as np
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    W = torch.randn((K, N), generator=gen, device="cuda") * 0.02
    Bq = ops.empty((K, N), np.int8)
    Bs = ops.empty((N,), np.float32)
    ops.lib().call("lhq_q8_quantize_per_col", W.data_ptr(), Bq.data_ptr(), Bs.data_ptr(), K, N, ops.stream())
    del W
    Bt = ops.prepack_b8(Bq, K, N)
    del Bq
    X = torch.randn((M, K), generator=gen, device="cuda")
    # 0.1 % of the activations replaced by +-20 outliers (config 3)
    n_out = max(1, (M * K) // 1000)
    pos = torch.randint(0, M * K, (n_out,), generator=gen, device="cuda")
    sign = torch.where(torch.rand((n_out,), generator=gen, device="cuda") < 0.5, -20.0, 20.0)
    X.view(-1)[pos] = sign
    Xb = X.to(torch.bfloat16).view(torch.int16)
    del X
    Aq = ops.empty((M, K), np.int8)
    As = ops.empty((M,), np.float32)
    C = ops.empty((M, N), np.int16)
    fn = ops.lib().cdll.lhq_gemm_w8a8_bf16
    qfn = ops.lib().cdll.lhq_q8_quantize_per_row_bf16

    def launch(_i):
        st = fn(Aq.data_ptr(), Bt.data_ptr(), As.data_ptr(), Bs.data_ptr(), C.data_ptr(), M, N, K, ops.stream())
        if st:
            raise RuntimeError(f"lhq_gemm_w8a8_bf16: {ops.lib().last_error()}")

    def qlaunch(_i):
        st = qfn(Xb.data_ptr(), Aq.data_ptr(), As.data_ptr(), M, K, ops.stream())
        if st:
            raise RuntimeError(f"lhq_q8_quantize_per_row_bf16: {ops.lib().last_error()}")

    qlaunch(0)
    torch.cuda.synchronize()
    timer = GraphTimer(launch, 1, chunk=16)
    ms, _ = timer.time(steps, warmup)
    us = ms * 1e3 / steps
    p50, p90 = timer.chunk_percentiles(steps)
    ops_per = 2 * M * K * N
    # the register-only MFMA rate on these same quantized values, with the
    # tile's instruction and order (v_mfma_i32_16x16x64_i8, one MFMA per
    # accumulator in turn: probe kind 6), and the same GEMM on all-zero
    # operands (the clock under the power limit depends on the values the
    # matrix cores multiply)
    same = operand_probe(ops, 6, Aq, Bt, iters=8000)
    Az = torch.zeros_like(Aq)
    Bz = torch.zeros_like(Bt)

    def zlaunch(_i):
        st = fn(Az.data_ptr(), Bz.data_ptr(), As.data_ptr(), Bs.data_ptr(), C.data_ptr(), M, N, K, ops.stream())
        if st:
            raise RuntimeError(f"lhq_gemm_w8a8_bf16: {ops.lib().last_error()}")

    zms, _ = GraphTimer(zlaunch, 1, chunk=16).time(steps, warmup)
    zus = zms * 1e3 / steps
    del Az, Bz
    qms, _ = GraphTimer(qlaunch, 1, chunk=16).time(steps, warmup)
    qus = qms * 1e3 / steps
    qbytes = M * K * 2 + M * K + M * 4
    # the per-output-channel weight quantizer (quant.cpp:75-96) on this B
    W = torch.randn((K, N), generator=gen, device="cuda") * 0.02
    Bq = ops.empty((K, N), np.int8)
    wfn = ops.lib().cdll.lhq_q8_quantize_per_col

    def wlaunch(_i):
        st = wfn(W.data_ptr(), Bq.data_ptr(), Bs.data_ptr(), K, N, ops.stream())
        if st:
            raise RuntimeError(f"lhq_q8_quantize_per_col: {ops.lib().last_error()}")

    wsteps = max(5, steps // 10)
    wms, _ = GraphTimer(wlaunch, 1, chunk=8).time(wsteps, 2)
    wus = wms * 1e3 / wsteps
    wbytes = K * N * 4 + K * N + N * 4
    del W, Bq
    res = {"M": M, "K": K, "N": N, "us_per_call": us, "tops": ops_per / (us * 1e-6) / 1e12,
           "act_quant_us": qus, "act_quant_gbs": qbytes / (qus * 1e-6) / 1e9,
           "weight_quant_us": wus, "weight_quant_gbs": wbytes / (wus * 1e-6) / 1e9}
    res["mfma_frac"] = res["tops"] / INT8_PEAK_TOPS
    res["us_p50_chunk"], res["us_p90_chunk"] = p50, p90
    res["sustained_same_operands"] = same
    res["frac_of_sustained"] = res["tops"] / same["value"]
    res["us_zero_operands"] = zus
    res["tops_zero_operands"] = ops_per / (zus * 1e-6) / 1e12
    del Bt, Xb, Aq, As, C
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def bench_8bit_small_m(ops, steps, warmup, seed=0, K=4096, N=14336, ms=(1, 17, 32, 64, 128, 256, 512), nsets=6):
    """W8A8 (bf16 output, and the reference's fp32 output with alpha = 1,
    beta = 0) and FP8 e4m3 at batched-decode row counts, timed over `nsets`
    rotating weight sets (6 x 58.7 MB at K=4096, N=14336, beyond the Infinity
    Cache); random int8 / e4m3 operands.  Bytes: K*N weight codes + M*K
    activations + 4 (M + N) scales + the output."""
    import numpy as np
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    L = ops.lib().cdll
    Bt8, Bs8, Bt_f8 = [], [], []
    for _ in range(nsets):
        W = torch.randn((K, N), generator=gen, device="cuda") * 0.02
        Bq = ops.empty((K, N), np.int8)
        Bs = ops.empty((N,), np.float32)
        ops.lib().call("lhq_q8_quantize_per_col", W.data_ptr(), Bq.data_ptr(), Bs.data_ptr(), K, N, ops.stream())
        Bt8.append(ops.prepack_b8(Bq, K, N))
        Bs8.append(Bs)
        del W, Bq
        # e4m3 codes below 0x70 (finite, |v| < 256), either sign
        f8 = torch.randint(0, 0x70, (K, N), dtype=torch.uint8, device="cuda", generator=gen)
        f8 |= (torch.randint(0, 2, (K, N), dtype=torch.uint8, device="cuda", generator=gen) << 7)
        Bt_f8.append(ops.prepack_b8(f8, K, N))
        del f8
    sa = torch.tensor([0.01], device="cuda")
    sb = torch.tensor([0.02], device="cuda")
    rows = []
    for M in ms:
        Aq = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=gen)
        As = torch.rand((M,), device="cuda", generator=gen) * 0.01
        A8 = torch.randint(0, 0x70, (M, K), dtype=torch.uint8, device="cuda", generator=gen)
        Cb = ops.empty((M, N), np.int16)
        Cf = torch.zeros((M, N), device="cuda")

        def w8_bf16(i):
            j = i % nsets
            st = L.lhq_gemm_w8a8_bf16(Aq.data_ptr(), Bt8[j].data_ptr(), As.data_ptr(), Bs8[j].data_ptr(),
                                      Cb.data_ptr(), M, N, K, ops.stream())
            if st:
                raise RuntimeError(ops.lib().last_error())

        def w8_f32(i):
            j = i % nsets
            st = L.lhq_gemm_w8a8(Aq.data_ptr(), Bt8[j].data_ptr(), As.data_ptr(), Bs8[j].data_ptr(), Cf.data_ptr(),
                                 M, N, K, 1.0, 0.0, ops.stream())
            if st:
                raise RuntimeError(ops.lib().last_error())

        def fp8(i):
            j = i % nsets
            st = L.lhq_gemm_fp8_e4m3(A8.data_ptr(), Bt_f8[j].data_ptr(), sa.data_ptr(), sb.data_ptr(), Cf.data_ptr(),
                                     M, N, K, 1.0, 0.0, ops.stream())
            if st:
                raise RuntimeError(ops.lib().last_error())

        row = {"M": M, "K": K, "N": N}
        for name, fn, ob in (("w8a8_bf16", w8_bf16, 2), ("w8a8_f32", w8_f32, 4), ("fp8_f32", fp8, 4)):
            ms_, _ = GraphTimer(fn, nsets, chunk=nsets * 8).time(steps, warmup)
            us = ms_ * 1e3 / steps
            byts = K * N + M * K + 4 * (M + N) + M * N * ob
            row[name] = {"us": round(us, 2), "gbs": round(byts / (us * 1e-6) / 1e9, 1),
                         "hbm_frac": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "tops": round(2.0 * M * K * N / (us * 1e-6) / 1e12, 1)}
        rows.append(row)
        del Aq, As, A8, Cb, Cf
    del Bt8, Bs8, Bt_f8
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return rows


def bench_w8_gemv(ops, steps, warmup, seed=0, K=4096, N=4096, min_rotate_bytes=2 * INFINITY_CACHE_BYTES + (1 << 26)):
    """Config 1: the W8 per-output-channel int8 GEMV through the reference's
    gemm_quant path (gemm_quant.cpp:29-49 at M=1).  One step is the
    reference's sequence: q8_quantize_per_row of the fp32 activation row
    (quant.cpp:52-63), then gemm_w8a8 with fp32 output, alpha = 1, beta = 0.
    Weights: fp32 N(0,0.02) [K,N] quantized per column on the device
    (quant.cpp:75-96) and prepacked once, rotated over sets beyond the
    Infinity Cache.  Also timed: the GEMV alone (the roofline figure, HBM:
    K*N int8 codes + 4N scales + K int8 + 4 row scale + 4N fp32 out)."""
    import numpy as np
    import torch
    M = 1
    gemv_bytes = K * N + 4 * N + M * K + 4 * M + 4 * M * N
    quant_bytes = 4 * M * K + M * K + 4 * M
    nsets = max(2, -(-min_rotate_bytes // (K * N)))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    sets = []
    for _ in range(nsets):
        W = torch.randn((K, N), generator=gen, device="cuda") * 0.02
        Bq = ops.empty((K, N), np.int8)
        Bs = ops.empty((N,), np.float32)
        ops.lib().call("lhq_q8_quantize_per_col", W.data_ptr(), Bq.data_ptr(), Bs.data_ptr(), K, N, ops.stream())
        del W
        sets.append((ops.prepack_b8(Bq, K, N), Bs))
        del Bq
    A = [torch.randn((M, K), generator=gen, device="cuda") for _ in range(nsets)]
    Aq = [ops.empty((M, K), np.int8) for _ in range(nsets)]
    As = [ops.empty((M,), np.float32) for _ in range(nsets)]
    C = [torch.zeros((M, N), device="cuda") for _ in range(nsets)]
    qfn = ops.lib().cdll.lhq_q8_quantize_per_row
    gfn = ops.lib().cdll.lhq_gemm_w8a8

    def gemv(j):
        st = gfn(Aq[j].data_ptr(), sets[j][0].data_ptr(), As[j].data_ptr(), sets[j][1].data_ptr(), C[j].data_ptr(),
                 M, N, K, 1.0, 0.0, ops.stream())
        if st:
            raise RuntimeError(f"lhq_gemm_w8a8: {ops.lib().last_error()}")

    def quant(j):
        st = qfn(A[j].data_ptr(), Aq[j].data_ptr(), As[j].data_ptr(), M, K, ops.stream())
        if st:
            raise RuntimeError(f"lhq_q8_quantize_per_row: {ops.lib().last_error()}")

    def step(i):
        quant(i % nsets)
        gemv(i % nsets)

    chunk = nsets * max(1, 64 // nsets)
    for j in range(nsets):
        quant(j)
    t_step = GraphTimer(step, nsets, chunk=chunk)
    ms_step, _ = t_step.time(steps, warmup)
    t_gemv = GraphTimer(lambda i: gemv(i % nsets), nsets, chunk=chunk)
    ms_gemv, _ = t_gemv.time(steps, warmup)
    p50, p90 = t_gemv.chunk_percentiles(steps)
    us_step = ms_step * 1e3 / steps
    us_gemv = ms_gemv * 1e3 / steps
    res = {"leg": "w8_gemv_config1", "M": M, "K": K, "N": N, "kernel": "gemm8_mid_kernel (16-row blocks)",
           "weights": "int8 per output channel (column) scales, prepacked once", "weight_sets": nsets,
           "rotate_bytes": nsets * K * N, "gemv_bytes": gemv_bytes,
           "us_per_step_quant_plus_gemv": round(us_step, 3), "us_per_gemv": round(us_gemv, 3),
           "us_per_gemv_p50_p90": [round(p50, 3), round(p90, 3)],
           "gemv_gbs": round(gemv_bytes / (us_gemv * 1e-6) / 1e9, 1),
           "step_gbs": round((gemv_bytes + quant_bytes) / (us_step * 1e-6) / 1e9, 1)}
    res["hbm_frac"] = round(res["gemv_gbs"] / HBM_PEAK_GBS, 4)
    del t_step, t_gemv, sets, A, Aq, As, C
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def diag_lib():
    """liblonghorn_diag.so: the matrix-core rate probes (not the product library)."""
    from longhornai_amd import capi
    return capi.load_diag()


PROBE_OPS_PER_MFMA = {0: 65536, 1: 131072, 2: 16384, 3: 65536, 4: 65536, 5: 32768, 6: 32768, 7: 32768}
PROBE_MFMAS_PER_ITER = {0: 32, 1: 32, 2: 32, 3: 32, 4: 64, 5: 64, 6: 32, 7: 32}


def operand_probe(ops, kind: int, A, B, iters: int = 4000, steps: int = 5, warmup: int = 2):
    """The matrix cores' rate on given operand values: lhd_probe_mfma_operands
    (the diagnostics library, include/longhorn_diag.h)
    with one workgroup of 4 waves per CU (one wave per SIMD, the W8A8 / FP8
    tiles' occupancy), each wave issuing MFMAs on 16 accumulators in turn from
    fragments it loaded once.  The fragments are bytes from the start of the
    device tensors A and B (A blocks from A, B blocks from B), so the figure is
    the register-only rate on the values a GEMM multiplies; the MFMA's power
    draw, and with it the clock under the power limit, depends on them.
    Returns the rate and the sustained shader clock (s_memtime over
    s_memrealtime ticks)."""
    import numpy as np
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    a = A.reshape(-1).view(torch.uint8)
    b = B.reshape(-1).view(torch.uint8)
    # [set][fragment: 4 A blocks, 4 B blocks][64 lanes x 16 bytes]; kind 1
    # takes the fragments' high halves from the next 8 KiB of each operand
    halves = []
    for h in range(2 if kind == 1 else 1):
        fa = a[h * 8192:(h + 1) * 8192].reshape(2, 4, 1024)
        fb = b[h * 8192:(h + 1) * 8192].reshape(2, 4, 1024)
        halves.append(torch.cat([fa, fb], dim=1).reshape(-1))
    buf = torch.zeros(32768, dtype=torch.uint8, device="cuda")
    src = torch.cat(halves)
    buf[:src.numel()] = src
    sink = ops.empty((cus,), np.int32)
    clocks = torch.zeros(2 * cus, dtype=torch.int64, device="cuda")

    def launch(_i):
        st = diag_lib().cdll.lhd_probe_mfma_operands(kind, buf.data_ptr(), cus, iters, sink.data_ptr(),
                                                    clocks.data_ptr(), ops.stream())
        if st:
            raise RuntimeError(f"lhd_probe_mfma_operands: {diag_lib().last_error()}")

    ms, _ = GraphTimer(launch, 1, chunk=steps).time(steps, warmup)
    rate = cus * 4 * iters * PROBE_MFMAS_PER_ITER[kind] * PROBE_OPS_PER_MFMA[kind] * steps / (ms * 1e-3) / 1e12
    c = clocks.view(cus, 2).double()
    ghz = float((c[:, 0] / c[:, 1]).mean()) * 0.1
    del buf, sink, clocks
    return {"value": round(rate, 1), "unit": "TOPS" if kind in (0, 3, 4, 5, 6, 7) else "TFLOPS", "ghz": round(ghz, 3),
            "us_per_launch": round(ms * 1e3 / steps, 1)}


def mfma_ceiling(ops, steps: int = 5, warmup: int = 2):
    """The matrix cores' sustained rate with every CU loaded: a probe kernel
    of back-to-back MFMAs on register operands (no memory traffic; four
    independent accumulators in turn, or one dependent chain), timed like the
    legs.  The GEMM legs' MFMA fractions are read against this as well as
    against the published peaks."""
    import numpy as np
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = ops.empty((8 * cus,), np.int32)
    out = {}
    # eight waves per SIMD (8 workgroups of 4 waves per CU), and the int8
    # 32x32x32 form also at one wave per SIMD, the W8A8 tile's occupancy
    for kind, name, per_op, iters, peak, blocks in (
            (0, "int8_32x32x32_one_wave", 65536, 22400, INT8_PEAK_TOPS, cus),
            (0, "int8_32x32x32", 65536, 2800, INT8_PEAK_TOPS, None),
            (3, "int8_16x16x64", 32768, 5600, INT8_PEAK_TOPS, None),
            (1, "bf16_16x16x32", 16384, 5600, BF16_PEAK_TFLOPS, None),
            (2, "bf16_32x32x16", 32768, 2800, BF16_PEAK_TFLOPS, None),
            (4, "bf16_16x16x32_valu2", 16384, 5600, BF16_PEAK_TFLOPS, None),
            (5, "bf16_16x16x32_valu4", 16384, 5600, BF16_PEAK_TFLOPS, None),
            (6, "bf16_16x16x32_chain", 16384, 5600, BF16_PEAK_TFLOPS, None),
            (7, "int8_16x16x64_chain", 32768, 5600, INT8_PEAK_TOPS, None)):
        blocks = 8 * cus if blocks is None else blocks
        def launch(i, kind=kind, iters=iters, blocks=blocks):
            st = diag_lib().cdll.lhd_probe_mfma_rate(kind, blocks, iters, sink.data_ptr(), ops.stream())
            if st:
                raise RuntimeError(f"lhd_probe_mfma_rate: {diag_lib().last_error()}")
        ms, _ = GraphTimer(launch, 1, chunk=steps).time(steps, warmup)
        per_launch = blocks * 4 * iters * 4 * per_op
        rate = per_launch * steps / (ms * 1e-3) / 1e12
        out[name] = {"value": round(rate, 1), "unit": "TOPS" if kind in (0, 3, 7) else "TFLOPS", "peak": peak,
                     "frac": round(rate / peak, 4), "us_per_launch": round(ms * 1e3 / steps, 1)}
    del sink
    # the W8A8 / FP8 tiles' order on operands from memory: uniformly random
    # bytes (bf16: N(0,1) values) and zero bytes, which bound the rate a GEMM's
    # own values give
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    rnd = torch.randint(0, 256, (2, 16384), dtype=torch.uint8, device="cuda", generator=gen)
    nrm = torch.randn((2, 8192), generator=gen, device="cuda").to(torch.bfloat16)
    zero = torch.zeros((2, 16384), dtype=torch.uint8, device="cuda")
    for kind, name, peak, data in ((0, "int8_32x32x32_tile_order", INT8_PEAK_TOPS, {"random": rnd, "zero": zero}),
                                   (1, "fp8_32x32x64_tile_order", FP8_PEAK_TFLOPS, {"random": rnd, "zero": zero}),
                                   (2, "bf16_16x16x32_tile_order", BF16_PEAK_TFLOPS, {"normal": nrm, "zero": zero}),
                                   (3, "int8_32x32x32_k_chain2", INT8_PEAK_TOPS, {"random": rnd}),
                                   (4, "int8_32x32x32_k_chain4", INT8_PEAK_TOPS, {"random": rnd}),
                                   (5, "int8_16x16x64_k_chain4", INT8_PEAK_TOPS, {"random": rnd, "zero": zero}),
                                   (6, "int8_16x16x64_tile_order", INT8_PEAK_TOPS, {"random": rnd}),
                                   (7, "int8_16x16x64_k_chain2", INT8_PEAK_TOPS, {"random": rnd})):
        for dn, d in data.items():
            r = operand_probe(ops, kind, d[0], d[1],
                              iters={0: 4000, 1: 2000, 2: 8000, 3: 4000, 4: 2000, 5: 4000, 6: 8000, 7: 8000}[kind])
            r.update(peak=peak, frac=round(r["value"] / peak, 4))
            out[f"{name}_{dn}"] = r
    del rnd, nrm, zero
    return out


def copy_probe(nbytes: int = 1 << 30, reps: int = 5) -> None:
    """A plain device copy of known size: the calibration kernel for the
    FETCH_SIZE / WRITE_SIZE counters (each launch reads and writes nbytes)."""
    import torch
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# CPU baseline (test infrastructure: the reference's path or its restatement)
# ---------------------------------------------------------------------------

def host_cpu() -> str:
    """The host CPU's model name and the cores this process may use."""
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return f"{model}; host nproc={os.cpu_count()}, {usable} usable by this process"


def cpu_baseline_w8a8(K: int, N: int, budget_s: float):
    """The reference's gemm_w8a8 (gemm_quant.cpp:29-49, fp32 output) on an
    M-slice of the W8A8 prefill workload.  Its rows are independent
    (gemm_quant.cpp:33), so the time per row extrapolates linearly to the
    M=4096 and M=2048 calls; the figure says so."""
    import numpy as np
    from oracle import Oracle, Ref, ref_available
    kind = "reference" if ref_available() else "port"
    impl = Ref() if kind == "reference" else Oracle()
    rng = np.random.default_rng(1)
    Bq = rng.integers(-127, 128, (K, N), dtype=np.int8)
    Bs = (rng.random(N, dtype=np.float32) + np.float32(0.5)) * np.float32(1e-3)

    def run(m):
        Aq = rng.integers(-127, 128, (m, K), dtype=np.int8)
        As = rng.random(m, dtype=np.float32) + np.float32(0.5)
        t0 = time.perf_counter()
        impl.gemm_w8a8(Aq, Bq, As, Bs)
        return time.perf_counter() - t0

    run(1)  # warm-up (touches B)
    t1 = run(1)
    m = max(1, min(64, int(budget_s / max(t1, 1e-6))))
    per_row = run(m) / m
    ops_row = 2 * K * N
    return {
        "value": ops_row / per_row / 1e12,
        "unit": "TOPS",
        "cores": 1,
        "kind": kind,
        "sample": (f"gemm_w8a8 (gemm_quant.cpp:29-49) on {m} rows of the K={K}, N={N} workload, "
                   f"{per_row * 1e3:.0f} ms/row, 1 thread; extrapolated linearly in M (rows are independent): "
                   f"M=4096 {4096 * per_row:.0f} s, M=2048 {2048 * per_row:.0f} s; {host_cpu()}"),
        "s_per_call_m4096_extrapolated": 4096 * per_row,
    }


def cpu_baseline(M: int, K: int, N: int, G: int, budget_s: float):
    import numpy as np
    from oracle import Oracle, Ref, ref_available
    kind = "reference" if ref_available() else "port"
    impl = Ref() if kind == "reference" else Oracle()
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((K, N), dtype=np.float32) * np.float32(0.02))
    Bp, Bs = impl.q4_quantize_groupwise(W, G)
    del W
    A = rng.standard_normal((M, K), dtype=np.float32)
    times = []
    impl.gemm_w4a16_groupwise(A, Bp, Bs, N, G)  # warm-up
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        impl.gemm_w4a16_groupwise(A, Bp, Bs, N, G)
        times.append(time.perf_counter() - t0)
    p50 = statistics.median(times)
    per = w4a16_sym_f32_bytes(M, K, N, G)
    return {
        "value": per / p50 / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        "sample": (f"gemm_w4a16_groupwise (gemm_quant.cpp:54-82) M={M} K={K} N={N} G={G}, fp32 A/C, "
                   f"symmetric int4 + fp32 scales ({per} algorithmic B/call); p50 of {len(times)} calls, "
                   f"{p50 * 1e3:.1f} ms/call, 1 thread; {host_cpu()}"),
        "ms_per_call": p50 * 1e3,
        "speedup_gpu_over_cpu": None,
    }


# ---------------------------------------------------------------------------
# traffic from the committed PMC summary
# ---------------------------------------------------------------------------

def committed_traffic(kernel_key: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated against a plain copy), as recorded in
    profiles/<kernel_key>_pmc.md on a line `traffic_bytes_per_launch: <int>`."""
    path = os.path.join(ROOT, "profiles", f"{kernel_key}_pmc.md")
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", text)
    return int(m.group(1)) if m else None


def prefill_legs(ops):
    """Configs 5 (W4A16 at M = 64 and 4096 on the K=8192, N=28672 target
    shape) and 4 (grouped MoE), timed like the decode leg."""
    out = []
    for m, steps in ((64, 500), (4096, 40)):
        log(f"w4a16 prefill M={m} K=8192 N=28672: {steps} steps")
        r = bench_w4a16(ops, m, 8192, 28672, 128, steps, max(5, steps // 10), workspace=True)
        tf = 2 * m * 8192 * 28672 / (r["us_per_call"] * 1e-6) / 1e12
        log(f"  {r['us_per_call']:.1f} us/call  {tf:.0f} TFLOPS ({100 * tf / BF16_PEAK_TFLOPS:.1f}% of bf16 peak), "
            f"{r['gbs']:.0f} GB/s ({100 * r['hbm_frac']:.1f}% of HBM peak)")
        out.append({"leg": "w4a16_prefill", "M": m, "K": 8192, "N": 28672, "G": 128,
                    "entry": r["entry"], "workspace_bytes": r["workspace_bytes"],
                    "us_per_call": round(r["us_per_call"], 2), "tflops": round(tf, 1),
                    "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4), "gbs": round(r["gbs"], 1),
                    "hbm_frac": round(r["hbm_frac"], 4)})
    log("moe grouped W4A16 (config 4): 200 steps")
    r = bench_moe(ops, 200, 20)
    log(f"  {r['us_per_call']:.1f} us/call  {r['tflops']:.0f} TFLOPS ({100 * r['mfma_frac']:.1f}% of bf16 peak), "
        f"{r['gbs']:.0f} GB/s")
    out.append({"leg": "moe_grouped_w4a16", **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}})
    out.append(moe_layer_leg(ops))
    return out


def config_sweep(ops, name, ms, kns, G=128):
    """W4A16 bf16 over a benchmark config's shapes: each (M, K, N) timed like
    the decode leg (rotating weight sets where one set fits in the Infinity
    Cache), reported against the HBM roofline (algorithmic bytes) and the
    bf16 MFMA roofline (2*M*K*N)."""
    out = []
    for m in ms:
        for k, n in kns:
            flops = 2 * m * k * n
            steps = 200 if m <= 64 else max(10, int(2e14 // flops))
            r = bench_w4a16(ops, m, k, n, G, steps, max(5, steps // 10), workspace=True)
            tf = flops / (r["us_per_call"] * 1e-6) / 1e12
            bound = "hbm" if r["gbs"] / HBM_PEAK_GBS >= tf / BF16_PEAK_TFLOPS else "mfma"
            out.append({"M": m, "K": k, "N": n, "workspace_bytes": r["workspace_bytes"],
                        "us_per_call": round(r["us_per_call"], 2),
                        "gbs": round(r["gbs"], 1), "hbm_frac": round(r["hbm_frac"], 4),
                        "tflops": round(tf, 1), "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4), "bound": bound})
            log(f"  {name} M={m} K={k} N={n}: {r['us_per_call']:.1f} us  {r['gbs']:.0f} GB/s "
                f"({100 * r['hbm_frac']:.1f}% HBM)  {tf:.0f} TFLOPS ({100 * tf / BF16_PEAK_TFLOPS:.1f}% bf16)")
    return out


CONFIG2 = ((1, 4, 16), ((4096, 4096), (4096, 11008), (11008, 4096)))
CONFIG5 = ((1, 8, 64, 4096), ((8192, 10240), (8192, 8192), (8192, 57344), (28672, 8192)))


def moe_layer_leg(ops, tokens=512):
    log(f"moe layer (config 4, Mixtral shapes, {tokens} tokens): dispatch, gate/up + SwiGLU, down, combine")
    r = bench_moe_layer(ops, 100, 10, T=tokens)
    for name, st in r["stages"].items():
        extra = f"  {st['tflops']:.0f} TFLOPS ({100 * st['mfma_frac']:.1f}%)" if "tflops" in st else ""
        log(f"  {name}: {st['us']:.1f} us  {st['gbs']:.0f} GB/s{extra}")
    log(f"  layer: {r['layer_us']:.1f} us ({r['tokens_per_s'] / 1e6:.2f} M tokens/s)")
    return {"leg": "moe_layer_w4a16", **r}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline timing")
    ap.add_argument("--no-w8a8", action="store_true", help="skip the W8A8 prefill leg")
    ap.add_argument("--w8a8-steps", type=int, default=200)
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a 1 GiB device copy (PMC calibration kernel)")
    ap.add_argument("--no-prefill", action="store_true", help="skip the W4A16 prefill and MoE legs")
    ap.add_argument("--only", choices=["w4a16", "w8a8", "prefill", "moe", "fp8", "configs", "mfma", "f32", "w8gemv",
                                      "thin", "grouped", "smallm"],
                    default=None,
                    help="run one leg only (profiling); prints that leg's summary, not the bench line")
    ap.add_argument("--moe-tokens", type=int, default=512,
                    help="tokens of the --only moe leg (512 = config 4; 1-4 run the grouped decode kernel)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}): "
              "this build has no multi-GPU path; the kernels shard along N with no collective "
              "(see the design notes).", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    from longhornai_amd import ops
    ops.lib()  # fails loudly when the HIP library is missing

    if args.copy_probe:
        copy_probe()

    M, K, N, G = 1, 8192, 28672, 128
    if args.only == "w8a8":
        for m in (4096, 2048):
            r = bench_w8a8(ops, m, 4096, 14336, args.w8a8_steps, max(10, args.w8a8_steps // 10))
            log(f"w8a8 M={m} K=4096 N=14336: {r['us_per_call']:.1f} us  {r['tops']:.0f} TOPS "
                f"({100 * r['mfma_frac']:.1f}% of int8 peak, {100 * r['frac_of_sustained']:.1f}% of the "
                f"{r['sustained_same_operands']['value']:.0f} TOPS the MFMAs sustain on these values at "
                f"{r['sustained_same_operands']['ghz']:.2f} GHz); zero operands {r['us_zero_operands']:.1f} us")
            print(json.dumps({"leg": "w8a8_prefill", **r}), flush=True)
        return 0
    if args.only == "thin":
        # the thin-grid W4A16 launches (split K across workgroups through the
        # workspace entry point): config 5 at M=64, config 2 at M=16
        for m, kns in ((64, CONFIG5[1]), (16, CONFIG2[1])):
            for k, n in kns:
                r = bench_w4a16(ops, m, k, n, G, 200, 20, workspace=True)
                log(f"w4a16 thin M={m} K={k} N={n}: {r['us_per_call']:.1f} us  {r['gbs']:.0f} GB/s "
                    f"({100 * r['hbm_frac']:.1f}% HBM), workspace {r['workspace_bytes']} B")
                print(json.dumps({"leg": "w4a16_thin", "M": m, "K": k, "N": n, "us_per_call": round(r["us_per_call"], 2),
                                  "gbs": round(r["gbs"], 1), "hbm_frac": round(r["hbm_frac"], 4),
                                  "workspace_bytes": r["workspace_bytes"]}), flush=True)
        return 0
    if args.only == "grouped":
        r = bench_moe(ops, 200, 20)
        log(f"moe grouped W4A16 (config 4): {r['us_per_call']:.1f} us  {r['tflops']:.0f} TFLOPS "
            f"({100 * r['mfma_frac']:.1f}% of bf16 peak)")
        print(json.dumps({"leg": "moe_grouped_w4a16", **r}), flush=True)
        return 0
    if args.only == "smallm":
        for r in bench_8bit_small_m(ops, 240, 24):
            log(f"8-bit GEMMs M={r['M']} K={r['K']} N={r['N']}: W8A8 bf16 {r['w8a8_bf16']['us']:.1f} us, "
                f"fp32 {r['w8a8_f32']['us']:.1f} us, FP8 {r['fp8_f32']['us']:.1f} us")
            print(json.dumps({"leg": "8bit_small_m", **r}), flush=True)
        return 0
    if args.only == "w8gemv":
        r = bench_w8_gemv(ops, 500, 50)
        log(f"w8 gemv config 1 M=1 K=4096 N=4096: gemv {r['us_per_gemv']:.2f} us ({r['gemv_gbs']:.0f} GB/s, "
            f"{100 * r['hbm_frac']:.1f}% of HBM peak); quant + gemv {r['us_per_step_quant_plus_gemv']:.2f} us")
        print(json.dumps(r), flush=True)
        return 0
    if args.only == "fp8":
        for m in (4096, 2048):
            r = bench_fp8(ops, m, 4096, 14336, args.w8a8_steps, max(10, args.w8a8_steps // 10))
            log(f"fp8 e4m3 GEMM M={m} K=4096 N=14336: {r['us_per_call']:.1f} us  {r['tflops']:.0f} TFLOPS "
                f"({100 * r['mfma_frac']:.1f}% of fp8 peak, {100 * r['frac_of_sustained']:.1f}% of the "
                f"{r['sustained_same_operands']['value']:.0f} TFLOPS the MFMAs sustain on these values); "
                f"zero operands {r['us_zero_operands']:.1f} us")
            print(json.dumps(r), flush=True)
        return 0
    if args.only == "mfma":
        print(json.dumps({"leg": "mfma_ceiling", **mfma_ceiling(ops)}), flush=True)
        return 0
    if args.only == "f32":
        # the reference interface: decode shapes on the integer decode and
        # 16-row kernels, prefill shapes on the tile kernel; thin shapes also
        # through the workspace entry point (K split across workgroups, the
        # lh:: drop-in's route)
        for m, k, n, st, ws in ((1, 8192, 28672, 500, False), (16, 8192, 28672, 200, False),
                                (16, 8192, 28672, 200, True), (4, 8192, 28672, 200, True),
                                (64, 8192, 8192, 200, True), (64, 8192, 8192, 100, False),
                                (256, 8192, 8192, 100, False), (1024, 8192, 8192, 40, False),
                                (4096, 8192, 8192, 20, False)):
            r = bench_w4a16_f32(ops, m, k, n, G, st, max(3, st // 10), workspace=ws)
            log(f"w4a16 fp32 interface M={m} K={k} N={n} ({r['entry']}): {r['us_per_call']:.1f} us  "
                f"{r['gbs']:.0f} GB/s ({100 * r['hbm_frac']:.1f}% HBM)  {r['tflops']:.0f} TFLOPS "
                f"({100 * r['mfma_frac']:.1f}% bf16)")
            print(json.dumps(r), flush=True)
        return 0
    if args.only == "configs":
        print(json.dumps({"leg": "w4a16_config2", "shapes": config_sweep(ops, "config 2", *CONFIG2)}), flush=True)
        print(json.dumps({"leg": "w4a16_config5", "shapes": config_sweep(ops, "config 5", *CONFIG5)}), flush=True)
        return 0
    if args.only == "moe":
        print(json.dumps(moe_layer_leg(ops, args.moe_tokens)), flush=True)
        return 0
    if args.only == "prefill":
        for r in prefill_legs(ops):
            print(json.dumps(r), flush=True)
        return 0
    log(f"w4a16 decode M={M} K={K} N={N} G={G}: {args.warmup} warmup + {args.steps} timed steps")
    w4 = bench_w4a16(ops, M, K, N, G, args.steps, args.warmup, direct=True)
    log(f"  {w4['us_per_call']:.2f} us/call  {w4['gbs']:.1f} GB/s  ({100 * w4['hbm_frac']:.1f}% of HBM peak), "
        f"{w4['weight_sets']} rotating sets = {w4['rotate_bytes'] / 2**20:.0f} MiB; per-launch time over "
        f"{w4['chunk_launches']}-launch chunks (a second pass): p50 {w4['us_p50_chunk']:.2f} us, "
        f"p90 {w4['us_p90_chunk']:.2f} us")

    if args.only == "w4a16":
        print(json.dumps({"leg": "w4a16_decode", **w4}), flush=True)
        return 0

    w8 = []
    if not args.no_w8a8:
        for m in (4096, 2048):
            log(f"w8a8 prefill M={m} K=4096 N=14336: {args.w8a8_steps} steps")
            r = bench_w8a8(ops, m, 4096, 14336, args.w8a8_steps, max(10, args.w8a8_steps // 10))
            log(f"  {r['us_per_call']:.1f} us/call  {r['tops']:.0f} TOPS ({100 * r['mfma_frac']:.1f}% of int8 peak); "
                f"act quant {r['act_quant_us']:.1f} us ({r['act_quant_gbs']:.0f} GB/s); "
                f"weight quant (per column) {r['weight_quant_us']:.1f} us ({r['weight_quant_gbs']:.0f} GB/s)")
            so = r["sustained_same_operands"]
            log(f"  register-only MFMAs on the same values: {so['value']:.0f} TOPS at {so['ghz']:.2f} GHz "
                f"(the GEMM reaches {100 * r['frac_of_sustained']:.1f}% of it); "
                f"the GEMM on zero operands: {r['us_zero_operands']:.1f} us ({r['tops_zero_operands']:.0f} TOPS)")
            w8.append(r)

    w8gemv = None
    if not args.no_w8a8:
        log("w8 gemv (config 1) M=1 K=4096 N=4096: 500 steps")
        w8gemv = bench_w8_gemv(ops, 500, 50)
        log(f"  gemv {w8gemv['us_per_gemv']:.2f} us ({w8gemv['gemv_gbs']:.0f} GB/s, {100 * w8gemv['hbm_frac']:.1f}% of "
            f"HBM peak); quant + gemv {w8gemv['us_per_step_quant_plus_gemv']:.2f} us")

    ceiling = None
    if not args.no_w8a8:
        ceiling = mfma_ceiling(ops)
        c8 = ceiling["int8_32x32x32_one_wave"]
        log(f"matrix-core ceiling (register-only MFMA probe, all CUs): int8 at one wave per SIMD {c8['value']:.0f} TOPS "
            f"({100 * c8['frac']:.1f}% of peak); bf16 {ceiling['bf16_16x16x32']['value']:.0f} TFLOPS "
            f"({100 * ceiling['bf16_16x16x32']['frac']:.1f}%)")
        cr = ceiling["int8_32x32x32_tile_order_random"]
        cz = ceiling["int8_32x32x32_tile_order_zero"]
        c6 = ceiling["int8_16x16x64_tile_order_random"]
        log(f"  int8 on operands from memory, in turn over accumulators: 32x32x32 random bytes {cr['value']:.0f} TOPS "
            f"at {cr['ghz']:.2f} GHz, zero bytes {cz['value']:.0f} TOPS at {cz['ghz']:.2f} GHz; 16x16x64 (the W8A8 "
            f"tile's form) random bytes {c6['value']:.0f} TOPS at {c6['ghz']:.2f} GHz")

    fp8 = []
    if not args.no_w8a8:
        log(f"fp8 e4m3 GEMM M=4096 K=4096 N=14336: {args.w8a8_steps} steps")
        r = bench_fp8(ops, 4096, 4096, 14336, args.w8a8_steps, max(10, args.w8a8_steps // 10))
        log(f"  {r['us_per_call']:.1f} us/call  {r['tflops']:.0f} TFLOPS ({100 * r['mfma_frac']:.1f}% of fp8 peak; "
            f"{100 * r['frac_of_sustained']:.1f}% of the {r['sustained_same_operands']['value']:.0f} TFLOPS the MFMAs "
            f"sustain on these values); zero operands {r['us_zero_operands']:.1f} us")
        fp8.append(r)

    pre = [] if args.no_prefill else prefill_legs(ops)

    cpu = cpu_w8 = None
    if not args.no_cpu:
        log(f"cpu baseline: ~{args.cpu_budget:.0f} s")
        cpu = cpu_baseline(M, K, N, G, args.cpu_budget)
        cpu["speedup_gpu_over_cpu"] = (cpu["ms_per_call"] * 1e3) / w4["us_per_call"]
        log(f"  {cpu['kind']}: {cpu['ms_per_call']:.1f} ms/call, {cpu['value']:.2f} GB/s")
        if w8:
            log(f"cpu baseline w8a8: ~{args.cpu_budget / 3:.0f} s")
            cpu_w8 = cpu_baseline_w8a8(4096, 14336, args.cpu_budget / 3)
            cpu_w8["speedup_gpu_over_cpu"] = cpu_w8["s_per_call_m4096_extrapolated"] * 1e6 / w8[0]["us_per_call"]
            log(f"  {cpu_w8['kind']}: {cpu_w8['value'] * 1e3:.2f} GOPS; {cpu_w8['sample']}")

    traffic = committed_traffic("w4a16_decode")
    line = {
        "metric": "W4A16 decode GB/s (% HBM peak) + W8A8 prefill TOPS (% MFMA peak), 1 GPU",
        "value": round(w4["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": w4["elapsed_ms"] / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 x bf16 -> bf16 (fp32 accumulate)",
        "data": "synthetic (seeded N(0,0.02) weights quantized on device, N(0,1) bf16 activations)",
        "config": {"workload": "w4a16_decode_gemv", "M": M, "K": K, "N": N, "group_size": G,
                   "weights": "asymmetric int4, fp16 scale + u4 zero per group",
                   "rotating_weight_sets": w4["weight_sets"], "rotate_bytes": w4["rotate_bytes"],
                   "bytes_per_step": w4["bytes_per_call"]},
        "roofline": {"bound": "hbm", "achieved": round(w4["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(w4["hbm_frac"], 4), "traffic": traffic,
                     "kernel": "w4_decode_i8_kernel", "algorithmic_bytes": w4["bytes_per_call"],
                     "us_per_launch": round(w4["us_per_call"], 3),
                     "us_per_launch_p50_p90": [round(w4["us_p50_chunk"], 3), round(w4["us_p90_chunk"], 3)],
                     "p50_p90_over": (f"{w4['chunk_launches']}-launch chunks of a second timed pass over "
                                      f"max(steps, 10 chunks) launches"),
                     "launch": ("direct stream launches enqueued while a spin kernel runs; the warm-up launches "
                                "run immediately before the opening event"),
                     "host_enqueue_ms": round(w4["host_enqueue_ms"], 3), "gpu_elapsed_ms": round(w4["elapsed_ms"], 3)},
        "w8a8_prefill": [
            {"M": r["M"], "K": r["K"], "N": r["N"], "us_per_call": round(r["us_per_call"], 2),
             "value": round(r["tops"], 1), "unit": "TOPS", "peak": INT8_PEAK_TOPS,
             "frac": round(r["mfma_frac"], 4), "act_quant_us": round(r["act_quant_us"], 2),
             "weight_quant_us": round(r["weight_quant_us"], 2), "weight_quant_gbs": round(r["weight_quant_gbs"], 1),
             "us_per_call_p50_p90": [round(r["us_p50_chunk"], 2), round(r["us_p90_chunk"], 2)],
             "sustained_same_operands": r["sustained_same_operands"],
             "frac_of_sustained": round(r["frac_of_sustained"], 4),
             "us_zero_operands": round(r["us_zero_operands"], 2)}
            for r in w8],
        "w8_gemv_config1": w8gemv,
        "mfma_ceiling": ceiling,
        "w8a8_cpu_baseline": cpu_w8,
        "fp8_gemm": fp8,
        "w4a16_prefill": pre,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

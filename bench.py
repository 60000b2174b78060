#!/usr/bin/env python3
"""Benchmark of the MI355X vk hot path (one GPU).

Headline (`value`): bf16 flash-attention forward + backward at B1 H16 S1024 D128 (the reference's attention
benchmark shape), in algorithmic TFLOP/s: 4*B*H*S^2*D forward + 2.5x that backward = 3.006e10 flop per
step (the convention of the reference's tools/bench_attention.py:39).  A step is what the reference's
benchmark times: F.scaled_dot_product_attention forward + backward through autograd on the vk device over
one batch already resident in HBM, which queues the hot path's three kernels (forward, dQ with the delta
pass folded in, dK/dV); W warm-up steps, then K steps between two synchronisations (wall clock, HIP events
beside it).  The three kernels queued directly through the hrt C ABI (no PyTorch) are reported beside it.
The roofline object belongs to the step's dominant kernel: its average duration over 200 back-to-back
launches between two events on the runtime stream, its HBM traffic from the rocprofv3 counter summary in
profiles/.  The same JSON line carries the other benchmark workloads (GEMMs, softmax, layer_norm, int8
dequant, the fused int8 linear, attention at S=4096, the DiT stack and block, image operators, ...) as
absolute TFLOP/s or GB/s and as a fraction of MI355X's published peaks, each timed after 25 ms of untimed
runs (its inputs are drawn on the CPU just before, and the idle GPU's clock needs milliseconds of load to
come back), and the CPU baseline: the reference's CPU path (torch CPU aten) at the full configuration,
with the other configurations and the oracle's float64 port beside it.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S] [--skip-cpu] [--only-attn]
       python bench.py --profile {fwd,dq,dkdv,copy,gemm,gemm1024,dq8,softmax,ln,dequant,dit} [--steps K]
                                                                   (launches only that workload, for rocprofv3)
       python bench.py --pmc-summary DIR [DIR ...]                 (per-kernel counters of rocprofv3 --pmc runs)
"""

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "torch-vulkan_amd"))

METRIC = "bf16 TFLOP/s flash-attn fwd+bwd (S1024,H16,D128) & GEMM; % of MFMA/HBM peak"
# MI355X dense bf16/f16 matrix peak: 256 CUs x 4096 flop/clock/CU x 2.4 GHz peak engine clock = 2516.6 TFLOP/s
# (AMD's published "2.5 PFLOP/s" dense figure; the 2:1-sparsity figures are never used here).  Every frac field
# of this file divides by this one constant.
PEAK_BF16_TFLOPS = 256 * 4096 * 2.4e9 / 1e12
PEAK_GBS = 8000.0  # MI355X HBM3E, published 8 TB/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only-attn", action="store_true", help="headline step only (for profiling runs)")
    ap.add_argument("--profile", choices=["fwd", "dq", "dkdv", "copy", "gemm", "gemm1024", "dq8", "softmax", "ln", "dequant",
                                          "dit", "ew", "reduce", "image", "dit_block"],
                    help="launch one kernel (or one benchmark workload) --steps times, untimed")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR", help="summarise rocprofv3 --pmc output directories")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(REPO, "profiles", "attn_traffic_s1024.txt")


def load_traffic(kernel):
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel of known size) from
    the committed rocprofv3 counter summary, or None when it has not been measured."""
    try:
        with open(TRAFFIC_FILE) as fh:
            for line in fh:
                f = line.split()
                if len(f) >= 3 and f[0] == kernel and f[1].startswith("hbm_bytes="):
                    return int(float(f[1].split("=", 1)[1]))
    except OSError:
        pass
    return None


def pmc_summary(dirs):
    """Average counter value per dispatch and kernel over rocprofv3 --pmc --output-format csv directories.
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are also given as bytes scaled by what the same counter reads
    for the 64 MiB device copy that `--profile copy` performs (bytes read = bytes written = 64 MiB)."""
    import csv
    import glob

    agg = {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
                agg.setdefault(name, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    avg = {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in agg.items()}
    copy = next((cs for k, cs in avg.items() if "ew_copy" in k or "copy_nd" in k), {})
    known_kib = 64 * 1024.0
    scale = {c: known_kib / copy[c] for c in ("FETCH_SIZE", "WRITE_SIZE") if copy.get(c)}
    for k, cs in sorted(avg.items()):
        print(f"== {k}")
        for c, v in sorted(cs.items()):
            extra = f"  scaled bytes {v * 1024 * scale[c]:.4g}" if c in scale else ""
            print(f"  {c:28s} {v:16.1f}{extra}")
    print("copy-kernel scale factors (64 MiB / counter):", {c: round(f, 4) for c, f in scale.items()})


def attn_flops(B, H, Sq, Sk, D):
    fwd = 4.0 * B * H * Sq * Sk * D
    return fwd, 2.5 * fwd


class Bench:
    def __init__(self, args):
        import torch

        import torch_vulkan
        from torch_vulkan import abi

        self.torch, self.tv, self.abi = torch, torch_vulkan, abi
        # autograd's backward inline on this thread (the training loop's thread), as a vk training script
        # would opt in: PyTorch otherwise hands the vk backward to a worker thread and waits for it
        torch_vulkan.set_inline_backward(True)
        self.rt = abi.Runtime()
        self.dev = torch.device("vk")
        self.args = args
        self.profile_n = 0  # > 0: time_graph only enqueues that many calls (rocprofv3 runs)

    # ---- helpers --------------------------------------------------------------------------------------
    def randn(self, shape, dtype, seed, scale=1.0):
        g = self.torch.Generator().manual_seed(seed)
        return (self.torch.randn(shape, generator=g) * scale).to(dtype).to(self.dev)

    SETTLE_S = 0.025

    def settle(self, launch):
        """Untimed launch() calls for at least 25 ms, in bursts of ~2 ms of GPU work each followed by a
        synchronisation (so the host never queues far ahead): every workload's inputs are drawn on the CPU
        just before it is timed, the GPU idles meanwhile, and its clock then needs milliseconds of load to
        come back up (the same kernel runs ~20% slower in the first milliseconds).  The warm-up time follows
        the default of triton.testing.do_bench (25 ms)."""
        rt = self.rt
        rt.event_record(8)
        launch()
        rt.event_record(9)
        burst = max(1, int(2.0 / max(rt.elapsed_ms(8, 9), 1e-3)))
        t_end = time.perf_counter() + self.SETTLE_S
        while time.perf_counter() < t_end:
            for _ in range(burst):
                launch()
            rt.synchronize()
        rt.synchronize()

    def time_graph(self, enqueue, reps, launches=3):
        """Average GPU time of one enqueue() call: a graph of `reps` calls, replayed `launches` times
        between two events on the runtime stream (after 25 ms of untimed replays, settle())."""
        rt = self.rt
        if self.profile_n:
            for i in range(self.profile_n):
                enqueue(i)
            rt.synchronize()
            return 1.0
        gid = rt.graph(lambda: [enqueue(i) for i in range(reps)])
        try:
            self.settle(lambda: rt.graph_launch(gid))
            rt.event_record(0)
            for _ in range(launches):
                rt.graph_launch(gid)
            rt.event_record(1)
            ms = rt.elapsed_ms(0, 1)
        finally:
            rt.graph_destroy(gid)
        return ms / (reps * launches)

    def time_direct(self, enqueue, reps, launches=3):
        """Average GPU time of one enqueue() call queued directly on the runtime stream: the launches of reps
        calls are collected once and queued with one hrt_dispatch_batch call per round (so Python's per-call
        cost does not stall the stream), launches rounds back to back between two events, after 25 ms of
        untimed rounds (settle())."""
        rt = self.rt
        pairs = []
        rt.dispatch = lambda name, args: pairs.append((name, args))  # collect instead of queueing
        try:
            for i in range(reps):
                enqueue(i)
        finally:
            del rt.dispatch
        b = rt.batch(pairs)
        self.settle(lambda: rt.run_batch(b))
        rt.event_record(0)
        for _ in range(launches):
            rt.run_batch(b)
        rt.event_record(1)
        rt.synchronize()
        return rt.elapsed_ms(0, 1) / (reps * launches)

    def time_best(self, enqueue, reps):
        """(ms, method): the faster of graph replay and direct queueing.  A graph node costs ~1.5 us of launch
        overhead; direct queueing costs host dispatch time, which only hides behind kernels longer than it."""
        if self.profile_n:
            return self.time_graph(enqueue, reps), "graph"
        g = self.time_graph(enqueue, reps)
        d = self.time_direct(enqueue, reps)
        return (g, "graph") if g <= d else (d, "direct")

    # ---- attention -----------------------------------------------------------------------------------
    def attn_setup(self, B, H, S, D, dtype="bf16"):
        torch, abi = self.torch, self.abi
        dt = torch.bfloat16 if dtype == "bf16" else torch.float16
        q, k, v, do = (self.randn((B, H, S, D), dt, s) for s in (1, 2, 3, 4))
        o = torch.empty((B, S, H, D), dtype=dt, device=self.dev)
        lse = torch.empty((B, H, S), dtype=torch.float32, device=self.dev)
        delta = torch.empty((B, H, S), dtype=torch.float32, device=self.dev)
        a = abi.AttnArgs()
        a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
        a.o, a.lse, a.dout, a.delta = o.data_ptr(), lse.data_ptr(), do.data_ptr(), delta.data_ptr()
        a.q_sb, a.q_sh, a.q_ss = q.stride(0), q.stride(1), q.stride(2)
        a.k_sb, a.k_sh, a.k_ss = k.stride(0), k.stride(1), k.stride(2)
        a.v_sb, a.v_sh, a.v_ss = v.stride(0), v.stride(1), v.stride(2)
        a.do_sb, a.do_sh, a.do_ss = do.stride(0), do.stride(1), do.stride(2)
        a.B, a.H, a.Sq, a.Sk, a.D = B, H, S, S, D
        a.scale = 1.0 / D ** 0.5
        # dQ computes delta = rowsum(O * dO) first (the shim's order: fwd, dQ + delta, dK/dV), and the
        # gradients take the inputs' layout, as the shim asks for dense inputs
        a.flags = abi.ATTN_GRAD_LIKE_INPUT
        dq, dk, dv = (torch.empty((B, H, S, D), dtype=dt, device=self.dev) for _ in range(3))
        a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
        ad = abi.AttnArgs.from_buffer_copy(a)
        ad.flags = abi.ATTN_GRAD_LIKE_INPUT | abi.ATTN_DQ_DELTA
        keep = (q, k, v, do, o, lse, delta, dq, dk, dv)
        names = {n: f"attn_{n}_mfma_{dtype}" for n in ("fwd", "dkdv", "dq")}

        def step(_i=0):
            self.rt.dispatch(names["fwd"], a)
            self.rt.dispatch(names["dq"], ad)
            self.rt.dispatch(names["dkdv"], a)

        kernels = {
            "fwd": lambda _i: self.rt.dispatch(names["fwd"], a),
            "dq": lambda _i: self.rt.dispatch(names["dq"], ad),
            "dkdv": lambda _i: self.rt.dispatch(names["dkdv"], a),
        }
        return step, kernels, keep, names

    def attn_headline(self):
        """The headline step, as the reference's tools/bench_attention.py:17-36 takes it: [B,S,H,D] bf16
        tensors viewed as [B,H,S,D] through transpose(1,2), F.scaled_dot_product_attention forward and
        backward through autograd on the vk device, W untimed warm-up steps, then K steps between two
        synchronisations (wall clock, and HIP events on the runtime stream beside it).

        Before it, the step's three kernels are each launched back to back, queued directly on the runtime
        stream as the shim queues them (one hrt_dispatch_batch call) between two events: each kernel's
        average launch duration, from which the roofline's achieved rate is taken (an event recorded between
        every two kernels would cost ~6 us of idle time per event on this runtime).  That work comes first
        because the GPU's clock rises over the first milliseconds of load (the same forward kernel runs
        ~17.5 us right after start-up and ~14.7 us a few milliseconds later), so the headline is the steady
        state of a training loop rather than a cold start; the kernel-only step (the three kernels queued
        directly, no PyTorch) is reported beside it."""
        import torch.nn.functional as F

        rt, args, torch = self.rt, self.args, self.torch
        B, H, S, D = 1, 16, 1024, 128
        step, kernels, keep, names = self.attn_setup(B, H, S, D)
        # the operator path's inputs are made here, before any timing: drawing them on the CPU takes tens of
        # milliseconds, and a GPU left idle that long drops its clock, which the W warm-up steps of a short
        # run do not recover (20 timed steps read 55-70 us per step that way, against 54-55 in steady state)
        bf = torch.bfloat16
        qb, kb, vb, gb = (self.randn((B, S, H, D), bf, s) for s in (1, 2, 3, 4))
        gt = gb.transpose(1, 2)

        def op_step():
            q, k, v = (t.transpose(1, 2).detach().requires_grad_(True) for t in (qb, kb, vb))
            F.scaled_dot_product_attention(q, k, v).backward(gt)

        # One operator step as set-up, also before any timing: the first F.scaled_dot_product_attention +
        # backward() of a process spends milliseconds on the host in one-time set-up (PyTorch's and the
        # shim's first calls) while the GPU idles and drops its clock; inside the W warm-up steps that stall
        # left the K timed steps on a clock still recovering (measured: 66, 61, 59, ... 53 us per step over
        # the first 500 steps after it).  Here the kernel timings below bring the clock back up afterwards.
        op_step()
        rt.synchronize()
        fwd_f, bwd_f = attn_flops(B, H, S, S, D)
        order = ("fwd", "dq", "dkdv")
        reps = max(args.steps, 200)
        per = {k: self.time_direct(kernels[k], reps, launches=2) for k in order}
        self.kernel_sum_ms = sum(per.values())
        # the kernel-only step: W warm-up, K timed, queued directly on the runtime stream
        for _ in range(args.warmup):
            step()
        rt.synchronize()
        rt.event_record(0)
        for _ in range(args.steps):
            step()
        rt.event_record(1)
        rt.synchronize()
        self.kernel_step_ms = rt.elapsed_ms(0, 1) / args.steps
        del keep

        # the operator path; device memory over the timed steps as tools/bench_attention.py:29-41 reports it
        # (the allocator's peak of live bytes after a reset, and the live bytes before the steps)
        for _ in range(args.warmup):
            op_step()
        rt.synchronize()
        self.tv.reset_peak_live_bytes()
        live0 = self.tv.live_bytes()
        rt.event_record(2)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            op_step()
        rt.event_record(3)
        rt.synchronize()
        wall = (time.perf_counter() - t0) / args.steps * 1e3
        self.op_gpu_ms = rt.elapsed_ms(2, 3) / args.steps
        self.op_mem = {"peak_live_bytes": int(self.tv.peak_live_bytes()), "live_bytes_before": int(live0),
                       "note": "torch_vulkan.peak_live_bytes() over the K timed operator steps after "
                               "reset_peak_live_bytes(), as tools/bench_attention.py:29-41; inputs q, k, v, dO "
                               "(4 x 4 MiB) are live before the steps"}
        kc = self.tv.kernel_counts()
        assert kc.get("aten::_scaled_dot_product_fused_attention_overrideable", 0) > 0, "the fused kernels did not run"

        unit = 2.0 * B * H * S * S * D  # one S x S x D product
        # S, dP are shared by dK/dV; dQ's S and dP are recomputation, and its delta pass is memory work
        algo = {"fwd": 2 * unit, "dkdv": 4 * unit, "dq": 1 * unit}
        kstats = {}
        for k, t in per.items():
            e = {"kernel": names[k], "avg_us": round(t * 1e3, 3), "algo_tflop": algo[k] / 1e12}
            e["tflops"] = round(algo[k] / (t * 1e-3) / 1e12, 2)
            e["frac_of_bf16_peak"] = round(e["tflops"] / PEAK_BF16_TFLOPS, 4)
            kstats[k] = e
        dom = max(order, key=lambda k: per[k])
        ach = algo[dom] / (per[dom] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": round(PEAK_BF16_TFLOPS, 1), "unit": "TFLOP/s",
                "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": load_traffic(names[dom]), "kernel": names[dom],
                "algo_flop_per_launch": algo[dom], "avg_launch_us": round(per[dom] * 1e3, 3),
                "timing": f"{reps} back-to-back direct launches between two events on the runtime stream, 2 rounds"}
        return wall, (fwd_f + bwd_f) / (wall * 1e-3) / 1e12, kstats, roof

    def attn_s4096(self):
        B, H, S, D = 1, 16, 4096, 128
        step, kernels, keep, _ = self.attn_setup(B, H, S, D)
        t, how = self.time_best(lambda i: step(), 3)
        f, b = attn_flops(B, H, S, S, D)
        per = {n: round(self.time_graph(kernels[n], 5) * 1e3, 2) for n in ("fwd", "dkdv", "dq")}
        del keep
        return {"ms": round(t, 4), "tflops": round((f + b) / (t * 1e-3) / 1e12, 2), "timing": how,
                "frac_of_bf16_peak": round((f + b) / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), "kernel_us": per}

    # ---- GEMM --------------------------------------------------------------------------------------
    def gemm(self, M, K, N, layout, bias=False):
        torch, abi = self.torch, self.abi
        a = self.randn((M, K), torch.bfloat16, 1)
        if layout == "nt":  # F.linear: x @ W^T with W [N, K] read through its transposed view
            w = self.randn((N, K), torch.bfloat16, 2)
            b_sk, b_sn = w.stride(1), w.stride(0)
        else:
            w = self.randn((K, N), torch.bfloat16, 2)
            b_sk, b_sn = w.stride(0), w.stride(1)
        c = torch.empty((M, N), dtype=torch.bfloat16, device=self.dev)
        bv = self.randn((N,), torch.bfloat16, 3)
        m = abi.MmArgs()
        m.a, m.b, m.c, m.bias = a.data_ptr(), w.data_ptr(), c.data_ptr(), bv.data_ptr()
        m.M, m.N, m.K, m.batch = M, N, K, 1
        m.a_sm, m.a_sk, m.b_sk, m.b_sn = a.stride(0), a.stride(1), b_sk, b_sn
        m.c_sm, m.c_sn = N, 1
        m.bias_sn = 1
        m.alpha, m.beta, m.has_bias = 1.0, 1.0 if bias else 0.0, 1 if bias else 0
        t, how = self.time_best(lambda i: self.rt.dispatch("mm_mfma_bf16", m), 10)
        fl = 2.0 * M * N * K
        return {"shape": f"{M}x{K}x{N}", "layout": layout, "bias": bias, "avg_us": round(t * 1e3, 2), "timing": how,
                "tflops": round(fl / (t * 1e-3) / 1e12, 2), "frac_of_bf16_peak": round(fl / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}

    def mm_ops(self, A, B, C, bias=None, alpha=1.0, beta=0.0, ws=None):
        """Argument blocks for C = alpha * A @ B + beta * bias on 2-D views (any strides), the way the shim
        queues them (csrc/shim/op_gemm.cpp: try_product): one "mm_mfma_bf16" launch, or, for products too narrow
        to fill the GPU with 64 x 64 tiles, the split-K pair "mm_mfma_bf16" (fp32 partials into ws) +
        "mm_reduce_bf16" with the shim's split rule."""
        abi = self.abi
        M, K = A.shape
        N = B.shape[1]
        m = abi.MmArgs()
        m.a, m.b, m.c = A.data_ptr(), B.data_ptr(), C.data_ptr()
        m.M, m.N, m.K, m.batch = M, N, K, 1
        m.a_sm, m.a_sk, m.b_sk, m.b_sn = A.stride(0), A.stride(1), B.stride(0), B.stride(1)
        m.c_sm, m.c_sn = C.stride(0), C.stride(1)
        m.alpha, m.beta = alpha, beta
        bsm = bsn = 0
        if bias is not None and beta != 0.0:
            bsm, bsn = (0, bias.stride(0)) if bias.dim() == 1 else (bias.stride(0), bias.stride(1))
            m.bias, m.bias_sm, m.bias_sn, m.has_bias = bias.data_ptr(), bsm, bsn, 1
        S = 1  # the shim's K-split rule (op_gemm.cpp: k_splits)
        if K % 64 == 0 and min(M, N) <= 16:
            tiles = -(-(M if N <= 16 else N) // 16)
            while tiles * S < 256 and K % (64 * 2 * S) == 0 and K // (2 * S) >= 1536:
                S *= 2
        elif K % 64 == 0 and min(M, N) <= 64:
            tiles = -(-M // 64) * -(-N // 64)
            while tiles * S * 2 <= 256 and (K // 64) % (S * 2) == 0 and K // (S * 2) >= 128:
                S *= 2
        elif K % 64 == 0:
            tiles = max((M // 128) * (N // 256) if M % 128 == 0 and N % 256 == 0 else 0,
                        (M // 256) * (N // 128) if M % 256 == 0 and N % 128 == 0 else 0)
            if 0 < tiles < 192:
                while tiles * S < 192 and K % (64 * 2 * S) == 0 and K // (2 * S) >= 1536:
                    S *= 2
                if tiles * S < 192:
                    S = 1
        if S == 1:
            return [("mm_mfma_bf16", m)]
        assert ws is not None and ws.numel() >= S * M * N, "split-K workspace too small"
        r = abi.MmReduceArgs()
        r.ws, r.c, r.bias = ws.data_ptr(), m.c, m.bias
        r.M, r.N, r.splits, r.c_sm, r.c_sn, r.bias_sm, r.bias_sn = M, N, S, m.c_sm, m.c_sn, bsm, bsn
        r.alpha, r.beta, r.has_bias = alpha, beta, m.has_bias
        m.K, m.batch = K // S, S
        m.a_sb, m.b_sb = m.K * m.a_sk, m.K * m.b_sk
        m.c, m.c_sb, m.c_sm, m.c_sn = ws.data_ptr(), M * N, N, 1
        m.bias = m.has_bias = m.bias_sm = m.bias_sn = 0
        m.alpha, m.beta, m.flags = 1.0, 0.0, abi.MM_F32_OUT
        return [("mm_mfma_bf16", m), ("mm_reduce_bf16", r)]

    def dit_lora_stack(self):
        """BASELINE C4: the DiT-block linear stack (QKV 2048->6144, out-proj 2048->2048, MLP 2048->8192->2048)
        at M = 1024 tokens, bf16, frozen base weights with bias and rank-16 LoRA factors.  One step = per layer
        y = x W^T + b, h = x A^T, y += h B^T (forward) and dx = g W, dB = g^T h, dh = g B, dA = dh^T x,
        dx += dh A (backward: dX for the base, the four LoRA products), every product queued as the shim
        queues it.  TFLOP/s counts the base GEMMs (2 x 1.0308e11) plus the LoRA products."""
        torch = self.torch
        bf, M, r = torch.bfloat16, 1024, 16
        layers = [(2048, 6144), (2048, 2048), (2048, 8192), (8192, 2048)]
        ws = torch.empty(4 * 1024 * 2048, dtype=torch.float32, device=self.dev)  # >= S * M * N of every split product
        ops, base_ops, keep, flops, base_flops = [], [], [], 0.0, 0.0
        for li, (fin, fout) in enumerate(layers):
            x = self.randn((M, fin), bf, 100 + li)
            W = self.randn((fout, fin), bf, 110 + li, 0.02)
            b = self.randn((fout,), bf, 120 + li, 0.02)
            A = self.randn((r, fin), bf, 130 + li, 0.02)
            Bl = self.randn((fout, r), bf, 140 + li, 0.01)
            g = self.randn((M, fout), bf, 150 + li)
            y = torch.empty((M, fout), dtype=bf, device=self.dev)
            h = torch.empty((M, r), dtype=bf, device=self.dev)
            dx = torch.empty((M, fin), dtype=bf, device=self.dev)
            dB = torch.empty((fout, r), dtype=bf, device=self.dev)
            dh = torch.empty((M, r), dtype=bf, device=self.dev)
            dA = torch.empty((r, fin), dtype=bf, device=self.dev)
            keep += [x, W, b, A, Bl, g, y, h, dx, dB, dh, dA]
            base = [self.mm_ops(x, W.t(), y, b, 1.0, 1.0, ws=ws), self.mm_ops(g, W, dx, ws=ws)]
            lora = [self.mm_ops(x, A.t(), h, ws=ws), self.mm_ops(h, Bl.t(), y, y, 1.0, 1.0),
                    self.mm_ops(g.t(), h, dB, ws=ws), self.mm_ops(g, Bl, dh, ws=ws), self.mm_ops(dh.t(), x, dA, ws=ws),
                    self.mm_ops(dh, A, dx, dx, 1.0, 1.0)]
            ops += base[0] + lora[0] + lora[1] + base[1] + lora[2] + lora[3] + lora[4] + lora[5]
            base_ops += base[0] + base[1]
            base_flops += 2 * (2.0 * M * fin * fout)
            flops += 2 * (2.0 * M * fin * fout) + 2.0 * M * r * fin * 3 + 2.0 * M * r * fout * 3
        run = lambda seq: [self.rt.dispatch(n, a) for n, a in seq]  # noqa: E731
        t, how = self.time_best(lambda i: run(ops), 3)
        tb, _ = self.time_best(lambda i: run(base_ops), 3)
        del keep
        return {"ms": round(t, 4), "tflops": round(flops / (t * 1e-3) / 1e12, 2),
                "frac_of_bf16_peak": round(flops / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                "flop": flops, "base_gemms_ms": round(tb, 4), "lora_ms": round(t - tb, 4), "timing": how,
                "launches": len(ops)}

    def dit_block(self):
        """One DiT block with LoRA through the PyTorch operator API on the vk device, forward + backward, at
        the production shape of the benchmark stack: 1024 tokens, C = 2048, 16 heads of 128, a 4C tanh-GELU
        MLP, AdaLN shift / scale / gate from a conditioning vector, LayerNorm without affine parameters, fused
        attention on [B, T, H, D] projections viewed as [B, H, T, D], rank-16 LoRA on the four linears
        (frozen base weights, trainable factors and input).  The reference drives such blocks from
        sd-scripts (tests/anima_on_vk.py:25-102); sd-scripts is absent here, so the block is written out.
        `ms` is the wall time per step (W warm-up steps, then K steps between synchronisations);
        `graph_replay_ms` replays one recorded step (every kernel the step queued, as a HIP graph), which adds
        a graph node's launch cost (~1.5 us) to each of the step's `kernels_per_step` kernels.  The share of
        the step the GPU spends in kernels is the sum of their durations over the wall time, from a rocprofv3
        kernel trace of `--profile dit_block` (which runs 3 warm-up steps, then N steps, and prints the wall
        time per step).  `cpu_fallbacks` lists operators that ran on the CPU during the timed steps."""
        import torch.nn.functional as F

        torch, rt, args = self.torch, self.rt, self.args
        bf = torch.bfloat16
        B, T, C, H, R = 1, 1024, 2048, 16, 16
        D = C // H
        P = {"ada_w": self.randn((6 * C, C), bf, 1, 0.02), "ada_b": self.randn((6 * C,), bf, 2, 0.02)}
        lin = (("qkv", C, 3 * C), ("proj", C, C), ("fc1", C, 4 * C), ("fc2", 4 * C, C))
        for i, (name, fin, fout) in enumerate(lin):
            P[name + "_w"], P[name + "_b"] = self.randn((fout, fin), bf, 10 + i, 0.02), self.randn((fout,), bf, 20 + i, 0.02)
            P[name + "_A"] = self.randn((R, fin), bf, 30 + i, 0.02).requires_grad_(True)
            P[name + "_B"] = self.randn((fout, R), bf, 40 + i, 0.01).requires_grad_(True)
        x0, c, g = self.randn((B, T, C), bf, 50), self.randn((B, C), bf, 51), self.randn((B, T, C), bf, 52)
        trainable = [P[n + s] for n, _, _ in lin for s in ("_A", "_B")]

        def lora(x, n):
            return F.linear(x, P[n + "_w"], P[n + "_b"]) + F.linear(F.linear(x, P[n + "_A"]), P[n + "_B"])

        def step():
            for t in trainable:
                t.grad = None
            x = x0.detach().requires_grad_(True)
            s1, sc1, g1, s2, sc2, g2 = F.linear(F.silu(c), P["ada_w"], P["ada_b"]).unsqueeze(1).chunk(6, dim=-1)
            h = F.layer_norm(x, (C,), eps=1e-6) * (1 + sc1) + s1
            q, k, v = lora(h, "qkv").view(B, T, 3, H, D).unbind(2)
            a = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
            y = x + g1 * lora(a.transpose(1, 2).reshape(B, T, C), "proj")
            h = F.layer_norm(y, (C,), eps=1e-6) * (1 + sc2) + s2
            out = y + g2 * lora(F.gelu(lora(h, "fc1"), approximate="tanh"), "fc2")
            out.backward(g)

        if self.profile_n:  # --profile dit_block: the steps alone, for a kernel trace
            for _ in range(3):
                step()
            rt.synchronize()
            t0 = time.perf_counter()
            for _ in range(self.profile_n):
                step()
            rt.synchronize()
            wall = (time.perf_counter() - t0) / self.profile_n * 1e3
            print(json.dumps({"dit_block_profile": {"warmup_steps": 3, "steps": self.profile_n,
                                                    "wall_ms_per_step": round(wall, 4)}}), file=sys.stderr, flush=True)
            return {}
        for _ in range(max(args.warmup, 3)):
            step()
        self.settle(step)
        n0 = self.tv.stats()["dispatch_n"]
        step()
        rt.synchronize()
        kernels = int(self.tv.stats()["dispatch_n"] - n0)
        self.tv.reset_fallback_counts()
        K = max(args.steps, 10)
        rt.event_record(4)
        t0 = time.perf_counter()
        for _ in range(K):
            step()
        rt.event_record(5)
        rt.synchronize()
        wall = (time.perf_counter() - t0) / K * 1e3
        events = rt.elapsed_ms(4, 5) / K
        fallbacks = self.tv.fallback_counts()
        # base products (forward and dX; the base weights are frozen) + LoRA products + attention (fwd + bwd)
        base = sum(2.0 * T * fin * fout for _, fin, fout in lin)
        flops = 2 * base + sum(2.0 * T * R * (fin + fout) * 3 for _, fin, fout in lin)
        flops += sum(attn_flops(B, H, T, T, D)) + 2 * (2.0 * B * C * 6 * C)
        out = {"ms": round(wall, 4), "ms_gpu_events": round(events, 4), "tflops": round(flops / (wall * 1e-3) / 1e12, 2),
               "flop": flops, "cpu_fallbacks": fallbacks, "steps": K, "kernels_per_step": kernels,
               "shape": {"tokens": T, "C": C, "heads": H, "head_dim": D, "mlp": 4 * C, "lora_rank": R}}
        # A recorded replay of the step (no host work) is reported beside the wall time as graph_replay_ms; a
        # replay pays ~1.5 us per graph node, so it is not a measure of GPU idle time (the sum of the kernels'
        # durations over the wall time, from a rocprofv3 kernel trace of --profile dit_block, is).
        try:
            gid = rt.graph(step)
        except RuntimeError as e:  # a step that waits for the GPU (a CPU fallback) cannot be recorded
            out["graph_replay_ms"] = None
            out["graph_replay_note"] = f"the step could not be recorded: {e}"
            return out
        try:
            # replays of the recorded step alone (no host work), after 25 ms of untimed replays: recording it
            # leaves the GPU idle long enough to drop its clock
            self.settle(lambda: rt.graph_launch(gid))
            rt.event_record(6)
            for _ in range(5):
                rt.graph_launch(gid)
            rt.event_record(7)
            rt.synchronize()
            busy = rt.elapsed_ms(6, 7) / 5
        finally:
            rt.graph_destroy(gid)
        out["graph_replay_ms"] = round(busy, 4)
        return out

    def dq8_linear(self, M):
        torch, abi = self.torch, self.abi
        N, K = 8192, 2048
        g = torch.Generator().manual_seed(9)
        q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(self.dev)
        s = (torch.rand(N, 1, generator=g) * 0.019 + 0.001).to(torch.bfloat16).expand(N, K // 64).contiguous().to(self.dev)
        x = self.randn((M, K), torch.bfloat16, 7)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=self.dev)
        a = abi.MmDq8Args()
        a.x, a.q, a.scale, a.y = x.data_ptr(), q.data_ptr(), s.data_ptr(), y.data_ptr()
        a.M, a.N, a.K, a.nblocks, a.x_sm, a.x_sk, a.alpha, a.beta = M, N, K, K // 64, K, 1, 1.0, 0.0
        ws = None
        if M >= 2048:  # as the shim does: dequantize once into a workspace, then the GEMM
            ws = torch.empty((N, K), dtype=torch.bfloat16, device=self.dev)
            a.ws = ws.data_ptr()
        t, how = self.time_best(lambda i: self.rt.dispatch("mm_dq8_bf16", a), 10)
        fl = 2.0 * M * N * K
        return {"M": M, "avg_us": round(t * 1e3, 2), "tflops": round(fl / (t * 1e-3) / 1e12, 2), "timing": how,
                "frac_of_bf16_peak": round(fl / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}

    # ---- bandwidth kernels: rotate over > 512 MB so the 256 MB MALL cannot serve them ------------
    def bw(self, name, nbytes, sets, make_args, kernels):
        """Average time of one launch rotating over `sets` input sets; at least 64 launches per timed round so
        that the start-up latency of a round stays out of the average for long kernels too."""
        args = [make_args(i) for i in range(sets)]
        reps = -(-max(2 * sets, 64) // sets) * sets
        t, how = self.time_best(lambda i: [self.rt.dispatch(k, args[i % sets][j]) for j, k in enumerate(kernels)], reps)
        return {"avg_us": round(t * 1e3, 3), "gbs": round(nbytes / (t * 1e-3) / 1e9, 1),
                "frac_of_hbm_peak": round(nbytes / (t * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes": nbytes, "timing": how}

    def softmax(self):
        torch, abi = self.torch, self.abi
        R, C = 16384, 1024
        xs = [self.randn((R, C), torch.float32, 10 + i, 2.0) for i in range(5)]
        ys = [torch.empty_like(x) for x in xs]
        gs = [self.randn((R, C), torch.float32, 20 + i) for i in range(5)]
        dxs = [torch.empty_like(x) for x in xs]

        def fa(i):
            a = abi.SoftmaxArgs()
            a.x, a.y, a.outer, a.R, a.inner = xs[i].data_ptr(), ys[i].data_ptr(), R, C, 1
            return [a]

        def ba(i):
            a = abi.SoftmaxArgs()
            a.y, a.g, a.dx, a.outer, a.R, a.inner = ys[i].data_ptr(), gs[i].data_ptr(), dxs[i].data_ptr(), R, C, 1
            return [a]

        n = R * C * 4
        return {"fwd": self.bw("softmax_fwd", 2 * n, 5, fa, ["softmax_fwd_f32"]),
                "bwd": self.bw("softmax_bwd", 3 * n, 4, ba, ["softmax_bwd_f32"])}

    def layer_norm(self):
        torch, abi = self.torch, self.abi
        R, D, sets = 1024, 2048, 64
        bf = torch.bfloat16
        w, b = self.randn((D,), bf, 2), self.randn((D,), bf, 3)
        xs = [self.randn((R, D), bf, 100 + i) for i in range(sets)]
        gs = [self.randn((R, D), bf, 200 + i) for i in range(sets)]
        ys = [torch.empty_like(x) for x in xs]
        dxs = [torch.empty_like(x) for x in xs]
        mu = torch.empty(R, dtype=torch.float32, device=self.dev)
        rs = torch.empty(R, dtype=torch.float32, device=self.dev)
        ws = torch.empty((self.abi.ln_chunks(R, D), 2, D), dtype=torch.float32, device=self.dev)
        dw, db = torch.empty(D, dtype=bf, device=self.dev), torch.empty(D, dtype=bf, device=self.dev)

        def fa(i):
            a = abi.LnArgs()
            a.x, a.y, a.mean, a.rstd, a.w, a.b, a.rows, a.D, a.eps = (xs[i].data_ptr(), ys[i].data_ptr(), mu.data_ptr(),
                                                                      rs.data_ptr(), w.data_ptr(), b.data_ptr(), R, D, 1e-5)
            return [a]

        def ba(i):
            a = abi.LnArgs()
            a.x, a.g, a.mean, a.rstd, a.w, a.dx, a.ws, a.dw, a.db, a.rows, a.D = (
                xs[i].data_ptr(), gs[i].data_ptr(), mu.data_ptr(), rs.data_ptr(), w.data_ptr(), dxs[i].data_ptr(),
                ws.data_ptr(), dw.data_ptr(), db.data_ptr(), R, D)
            return [a]

        fwd_b = 2 * R * D * 2 + 2 * D * 2 + 2 * R * 4
        bwd_b = 3 * R * D * 2 + D * 2 + 2 * R * 4 + 2 * D * 2
        fwd = self.bw("ln_fwd", fwd_b, sets, fa, ["ln_fwd_bf16"])
        bwd = self.bw("ln_bwd", bwd_b, sets, ba, ["ln_bwd_bf16"])  # dx, then dw and db (two kernels)
        fwd["copy_floor"] = self.copy_floor(R * D * 2, R * D * 2, sets)
        bwd["copy_floor"] = self.copy_floor(2 * R * D * 2, R * D * 2, sets)
        return {"fwd": fwd, "bwd": bwd}

    def dequant(self):
        torch, abi = self.torch, self.abi
        R, C, sets = 8192, 2048, 24
        qs, ss, outs = [], [], []
        for i in range(sets):
            g = torch.Generator().manual_seed(i)
            qs.append(torch.randint(-127, 128, (R, C), generator=g, dtype=torch.int8).to(self.dev))
            ss.append((torch.rand(R, 1, generator=g) * 0.019 + 0.001).to(torch.bfloat16).expand(R, C // 64).contiguous().to(self.dev))
            outs.append(torch.empty((R, C), dtype=torch.bfloat16, device=self.dev))

        def mk(i):
            a = abi.Dq8Args()
            a.q, a.scale, a.out, a.rows, a.cols, a.nblocks = qs[i].data_ptr(), ss[i].data_ptr(), outs[i].data_ptr(), R, C, C // 64
            return [a]

        nbytes = R * C + R * (C // 64) * 2 + R * C * 2
        out = self.bw("dq8", nbytes, sets, mk, ["dq8_bf16"])
        out["copy_floor"] = self.copy_floor(R * C + R * (C // 64) * 2, R * C * 2, sets)
        return out

    def copy_floor(self, read_bytes, write_bytes, sets):
        """The runtime's own device copy (ew_copy, 16 bytes per lane) moving the same total bytes as a
        bandwidth kernel (half read, half written), timed the same way and rotating over as many buffers: the
        practical floor that kernel is compared with, launch cost included."""
        torch, abi = self.torch, self.abi
        n = (read_bytes + write_bytes) // 2 // 16 * 4  # fp32 elements, whole 16-byte chunks
        srcs = [torch.empty(n, dtype=torch.float32, device=self.dev).fill_(1.0) for _ in range(sets)]
        dsts = [torch.empty_like(x) for x in srcs]

        def mk(i):
            a = abi.CopyArgs()
            a.dst, a.src, a.ndim, a.dst_dtype, a.src_dtype = dsts[i].data_ptr(), srcs[i].data_ptr(), 1, 0, 0
            a.sizes[0], a.dst_strides[0], a.src_strides[0] = n, 1, 1
            return [a]

        r = self.bw("ew_copy", 2 * n * 4, sets, mk, ["ew_copy"])
        r["read_bytes"] = r["write_bytes"] = n * 4
        return r

    def elementwise(self):
        """ew_map at the shapes of the LoRA/DiT training step: the MLP activation forward and backward
        ([1024, 8192] bf16, tanh GELU), a bias add broadcast over rows, an optimizer moment update (lerp_ on
        16 M fp32 parameters) and a large flat bf16 add.  Every case rotates over enough buffers to exceed
        the 256 MB last-level cache; bytes are the compulsory HBM traffic (each operand read once, the
        output written once)."""
        torch, abi = self.torch, self.abi
        bf, f32 = torch.bfloat16, torch.float32
        dt = {bf: abi.BF16, f32: abi.F32}

        def ew(op, out, a, b=None, s0=0.0, bstrides=None):
            A = abi.EwArgs()
            A.op, A.out, A.a, A.out_dtype, A.a_dtype, A.s0 = abi.EW_OPS[op], out.data_ptr(), a.data_ptr(), dt[out.dtype], dt[a.dtype], s0
            A.ndim = out.dim()
            for i in range(out.dim()):
                A.sizes[i], A.out_strides[i], A.a_strides[i] = out.shape[i], out.stride(i), a.stride(i)
            if b is not None:
                A.b, A.b_dtype = b.data_ptr(), dt[b.dtype]
                for i, st in enumerate(bstrides or b.stride()):
                    A.b_strides[i] = st
            return A

        def case(name, shape, dtype, op, sets, nin, s0=0.0, bshape=None):
            n = 1
            for d in shape:
                n *= d
            es = torch.tensor([], dtype=dtype).element_size()
            xs = [[self.randn(shape if j == 0 or bshape is None else bshape, dtype, 40 + 10 * i + j) for j in range(nin)]
                  for i in range(sets)]
            outs = [torch.empty(shape, dtype=dtype, device=self.dev) for _ in range(sets)]

            def mk(i):
                a = xs[i][0]
                if nin == 1:
                    return [ew(op, outs[i], a, s0=s0)]
                b = xs[i][1]
                lead = len(shape) - b.dim()  # b broadcasts right-aligned over the leading dimensions
                bst = [0 if k < lead or b.shape[k - lead] == 1 else b.stride(k - lead) for k in range(len(shape))]
                return [ew(op, outs[i], a, b, s0=s0, bstrides=bst)]

            bbytes = n * es if bshape is None else (xs[0][1].numel() * es if nin > 1 else 0)
            nbytes = n * es * 2 + (bbytes if nin > 1 else 0)
            r = self.bw("ew_map", nbytes, sets, mk, ["ew_map"])
            r["op"] = op
            r["shape"] = list(shape)
            r["dtype"] = str(dtype).replace("torch.", "")
            return name, r

        cases = [
            case("gelu_tanh_fwd", (1024, 8192), bf, "gelu_tanh", 16, 1),
            case("gelu_tanh_bwd", (1024, 8192), bf, "gelu_tanh_bwd", 12, 2),
            case("bias_add_rows", (1024, 8192), bf, "add", 16, 2, s0=1.0, bshape=(8192,)),
            case("lerp_f32_16M", (16 * 1024 * 1024,), f32, "lerp_s", 3, 2, s0=0.1),
            case("add_bf16_64M", (8192, 8192), bf, "add", 2, 2, s0=1.0),
        ]
        return dict(cases)

    def reductions(self):
        """reduce_sum at the step's shapes: the bias gradient of the DiT MLP up-projection (sum over 1024
        rows of [1024, 8192] bf16), row sums of the softmax benchmark's [16384, 1024] fp32, a full sum of
        64 M fp32; and cat of three [1024, 2048] bf16 parts along the last dimension (three ew_copy launches
        into the slices).  Bytes: input read once + output written once."""
        import ctypes

        torch, abi = self.torch, self.abi
        dt = {torch.bfloat16: abi.BF16, torch.float32: abi.F32}

        def case(shape, dtype, mask, sets, seed):
            xs = [self.randn(shape, dtype, seed + i) for i in range(sets)]
            kept = [n for d, n in enumerate(shape) if not (mask >> d) & 1]
            n_out = 1
            for n in kept:
                n_out *= n
            outs = [torch.empty(kept, dtype=dtype, device=self.dev) for _ in range(sets)]

            def args(i):
                a = abi.ReduceArgs()
                a.x, a.out, a.ndim, a.x_dtype, a.out_dtype, a.reduce_mask, a.div = (
                    xs[i].data_ptr(), outs[i].data_ptr(), len(shape), dt[dtype], dt[dtype], mask, 1.0)
                for d, n in enumerate(shape):
                    a.sizes[d], a.strides[d] = n, xs[i].stride(d)
                return a

            wsn = self.rt.lib.hrt_reduce_workspace(ctypes.byref(args(0)))
            ws = torch.empty(max(wsn, 1), dtype=torch.float32, device=self.dev)

            def mk(i):
                a = args(i)
                a.ws = ws.data_ptr() if wsn > 0 else 0
                return [a]

            es = xs[0].element_size()
            r = self.bw("reduce_sum", xs[0].numel() * es + n_out * es, sets, mk, ["reduce_sum"])
            r["shape"], r["reduce_mask"], r["dtype"], r["workspace_floats"] = list(shape), mask, str(dtype)[6:], wsn
            return r

        R, C = 1024, 2048
        parts = [[self.randn((R, C), torch.bfloat16, 90 + 3 * i + j) for j in range(3)] for i in range(8)]
        cats = [torch.empty((R, 3 * C), dtype=torch.bfloat16, device=self.dev) for _ in range(8)]

        def cat_args(i):  # one "cat_rows16" launch, as the shim queues torch.cat of these parts
            a = abi.CatArgs()
            a.out, a.outer, a.out_row_bytes, a.nparts = cats[i].data_ptr(), R, 3 * C * 2, 3
            for j in range(3):
                a.src[j], a.row_bytes[j], a.col[j] = parts[i][j].data_ptr(), C * 2, j * C * 2
            return [a]

        cat = self.bw("cat_rows16", 2 * 3 * R * C * 2, 8, cat_args, ["cat_rows16"])
        cat["launches"] = 1
        return {"bias_grad_sum0_bf16_1024x8192": case((1024, 8192), torch.bfloat16, 0b01, 16, 300),
                "row_sum_f32_16384x1024": case((16384, 1024), torch.float32, 0b10, 5, 320),
                "full_sum_f32_64M": case((64 * 1024 * 1024,), torch.float32, 0b1, 2, 340),
                "cat_bf16_3x1024x2048_dim1": cat}

    def image_ops(self):
        """VAE-decoder shaped operators through PyTorch on the vk device (the adapters' host work included):
        conv3x3 512 -> 512 channels at 64x64 bf16 forward and forward + input gradient (the direct implicit
        GEMM), group_norm (32 groups) forward / backward on [1, 512, 128, 128] bf16, nearest x2 upsampling of
        [1, 512, 64, 64] bf16 forward / backward.  GPU time from events around 20 calls after 25 ms of
        untimed calls (settle())."""
        torch, rt = self.torch, self.rt
        import torch.nn.functional as F

        def gpu_ms(fn, n=20):
            self.settle(fn)
            rt.event_record(2)
            for _ in range(n):
                fn()
            rt.event_record(3)
            rt.synchronize()
            return rt.elapsed_ms(2, 3) / n

        bf = torch.bfloat16
        x = self.randn((1, 512, 64, 64), bf, 60)
        w = self.randn((512, 512, 3, 3), bf, 61, 0.02)
        go = self.randn((1, 512, 64, 64), bf, 62)
        flop = 2.0 * 512 * 512 * 9 * 64 * 64
        t_conv = gpu_ms(lambda: F.conv2d(x, w, None, padding=1))

        def conv_fb():
            xx = x.detach().requires_grad_(True)
            F.conv2d(xx, w, None, padding=1).backward(go)

        t_conv_fb = gpu_ms(conv_fb)  # forward + input gradient (frozen weights)
        xg = self.randn((1, 512, 128, 128), bf, 63)
        gw, gb = self.randn((512,), bf, 64), self.randn((512,), bf, 65)
        gg = self.randn((1, 512, 128, 128), bf, 66)
        t_gn = gpu_ms(lambda: F.group_norm(xg, 32, gw, gb, 1e-6))
        _, mean, rstd = torch.native_group_norm(xg, gw, gb, 1, 512, 128 * 128, 32, 1e-6)
        t_gnb = gpu_ms(lambda: torch.ops.aten.native_group_norm_backward(gg, xg, mean, rstd, gw, 1, 512, 128 * 128, 32,
                                                                       [True, True, True]))
        t_up = gpu_ms(lambda: F.interpolate(x, scale_factor=2, mode="nearest"))
        t_upb = gpu_ms(lambda: torch.ops.aten.upsample_nearest2d_backward(gg, [128, 128], [1, 512, 64, 64]))
        n_gn = 512 * 128 * 128 * 2
        return {"conv3x3_512_64x64_fwd": {"ms": round(t_conv, 4), "tflops": round(flop / t_conv / 1e9, 1)},
                "conv3x3_512_64x64_fwd_dx": {"ms": round(t_conv_fb, 4), "tflops": round(2 * flop / t_conv_fb / 1e9, 1)},
                "group_norm_fwd_1x512x128x128": {"ms": round(t_gn, 4), "gbs": round(2 * n_gn / t_gn / 1e6, 1)},
                "group_norm_bwd_1x512x128x128": {"ms": round(t_gnb, 4), "gbs": round(4 * n_gn / t_gnb / 1e6, 1)},
                "upsample2x_fwd_1x512x64x64": {"ms": round(t_up, 4), "gbs": round(5 * n_gn / 4 / t_up / 1e6, 1)},
                "upsample2x_bwd_1x512x64x64": {"ms": round(t_upb, 4), "gbs": round(5 * n_gn / 4 / t_upb / 1e6, 1)}}

    def transfers(self):
        """The block-swap path: host -> device bandwidth for 100 MB (about one DiT block's bf16 weights:
        QKV 2048x6144, out 2048x2048, MLP 2048x8192 and 8192x2048) from pageable memory (synchronous, what
        the reference does), from pinned memory synchronously, and asynchronously (hrt_upload_async on the
        copy stream); then the same asynchronous upload queued beside a run of 1024x2048x8192 bf16 GEMMs
        that does not touch its destination, against each alone: overlap = (t_gemm + t_upload - t_both) /
        min(t_gemm, t_upload).  Host wall-clock around a synchronize, median of 5."""
        import ctypes

        torch, abi, rt, lib = self.torch, self.abi, self.rt, self.rt.lib
        n = 100 * 1000 * 1000
        dev = torch.empty(n, dtype=torch.uint8, device=self.dev)
        pageable = torch.ones(n, dtype=torch.uint8)
        pin = lib.hrt_host_alloc(n)
        if not pin:
            raise RuntimeError("hrt_host_alloc failed: " + rt.last_error())
        ctypes.memset(pin, 1, n)

        def wall(fn, reps=5):
            ts = []
            for _ in range(reps + 1):
                rt.synchronize()
                t0 = time.perf_counter()
                fn()
                rt.synchronize()
                ts.append(time.perf_counter() - t0)
            return statistics.median(ts[1:])

        t_pg = wall(lambda: rt.check(lib.hrt_upload(dev.data_ptr(), pageable.data_ptr(), n), "upload"))
        t_ps = wall(lambda: rt.check(lib.hrt_upload(dev.data_ptr(), pin, n), "upload"))
        t_pa = wall(lambda: rt.check(lib.hrt_upload_async(dev.data_ptr(), pin, n), "upload_async"))
        M, K, N = 1024, 2048, 8192
        a, w = self.randn((M, K), torch.bfloat16, 1), self.randn((N, K), torch.bfloat16, 2)
        c = torch.empty((M, N), dtype=torch.bfloat16, device=self.dev)
        m = abi.MmArgs()
        m.a, m.b, m.c = a.data_ptr(), w.data_ptr(), c.data_ptr()
        m.M, m.N, m.K, m.batch = M, N, K, 1
        m.a_sm, m.a_sk, m.b_sk, m.b_sn, m.c_sm, m.c_sn = K, 1, 1, K, N, 1
        m.alpha = 1.0
        reps = max(1, int(t_pa / 40e-6))  # GEMMs (~40 us each) worth about one upload
        b = rt.batch([("mm_mfma_bf16", m)] * reps)
        t_gemm = wall(lambda: rt.run_batch(b))

        def both():
            rt.check(lib.hrt_upload_async(dev.data_ptr(), pin, n), "upload_async")
            rt.run_batch(b)

        t_both = wall(both)
        lib.hrt_host_free(pin)
        gbs = lambda t: round(n / t / 1e9, 2)  # noqa: E731
        return {"bytes": n, "pageable_sync_gbs": gbs(t_pg), "pinned_sync_gbs": gbs(t_ps), "pinned_async_gbs": gbs(t_pa),
                "gemm_ms": round(t_gemm * 1e3, 3), "gemms": reps, "upload_async_ms": round(t_pa * 1e3, 3),
                "both_ms": round(t_both * 1e3, 3),
                "overlap": round((t_gemm + t_pa - t_both) / min(t_gemm, t_pa), 3)}

    # ---- CPU baseline: the reference's CPU path (torch CPU aten) -------------------------------------
    def profile(self, which, n):
        """Launch one kernel of the headline step (or a 64 MiB device copy) n times and return: the workload
        that rocprofv3 --kernel-trace / --pmc runs wrap."""
        torch = self.torch
        workloads = {"gemm": lambda: self.gemm(1024, 2048, 8192, "nt"), "gemm1024": lambda: self.gemm(1024, 1024, 1024, "nn", True),
                     "dq8": lambda: self.dq8_linear(1024), "softmax": self.softmax, "ln": self.layer_norm,
                     "dequant": self.dequant, "dit": self.dit_lora_stack, "ew": self.elementwise,
                     "reduce": self.reductions, "image": self.image_ops, "dit_block": self.dit_block}
        if which in workloads:
            self.profile_n = n
            workloads[which]()
            self.profile_n = 0
        elif which == "copy":  # the runtime's own ew_copy kernel over 64 MiB: the counters' calibration
            abi = self.abi
            src = torch.empty(16 * 1024 * 1024, dtype=torch.float32, device=self.dev).fill_(1.0)
            dst = torch.empty_like(src)
            a = abi.CopyArgs()
            a.dst, a.src, a.ndim, a.dst_dtype, a.src_dtype = dst.data_ptr(), src.data_ptr(), 1, 0, 0
            a.sizes[0], a.dst_strides[0], a.src_strides[0] = src.numel(), 1, 1
            for _ in range(n):
                self.rt.dispatch("ew_copy", a)
        else:
            step, kernels, keep, _ = self.attn_setup(1, 16, 1024, 128)
            step()  # fwd, dQ (+delta), dK/dV once so that every input of the profiled kernel is valid
            for i in range(n):
                kernels[which](i)
        self.rt.synchronize()

    def cpu_baseline(self):
        """The reference's CPU path: torch's CPU aten operators, which are what the reference runs for anything
        its device does not take and what its tests compare against (tests/test_fused_attention.py,
        tests/test_mm.py, tests/test_rows.py, tests/test_dequant_int8.py), timed on this host with torch's
        thread pool.  `value` is the headline: F.scaled_dot_product_attention forward + backward in bf16 at the
        full [1,16,1024,128] configuration, in the same algorithmic TFLOP/s as the GPU step (the convention of
        tools/bench_attention.py:39-41).  `configs` times the other benchmark configurations the same way
        (GEMMs in TFLOP/s; softmax, layer_norm and dequant in GB/s of algorithmic bytes, as
        tools/bench_dequant_int8.py:28-29 counts them).  `oracle_port` is the float64 numpy restatement the
        parity tests check against, on 2 of the 16 heads.  Each figure is the median of at least 5 runs after
        one untimed run, within a time budget."""
        import numpy as np
        import torch
        import torch.nn.functional as F

        sys.path.insert(0, REPO)
        import oracle

        def median_time(fn, budget, at_least=5, at_most=200):
            fn()
            times = []
            t_end = time.perf_counter() + budget
            while len(times) < at_least or (time.perf_counter() < t_end and len(times) < at_most):
                t0 = time.perf_counter()
                fn()
                times.append(time.perf_counter() - t0)
            return statistics.median(times), len(times)

        model = ""
        try:  # the model name, plus family / model / stepping (a VM may report only "AMD EPYC")
            with open("/proc/cpuinfo") as fh:
                info = {}
                for l in fh:
                    if ":" in l:
                        k_, v_ = (x.strip() for x in l.split(":", 1))
                        info.setdefault(k_, v_)
                    elif info:
                        break
            model = info.get("model name", "")
            fam = [f"{k_} {info[k_]}" for k_ in ("cpu family", "model", "stepping") if k_ in info]
            if fam:
                model += " (" + ", ".join(fam) + ")"
        except OSError:
            pass
        # every core this process may run on (the headline and the other configurations); torch's default
        # pool (OMP_NUM_THREADS) is timed beside the headline
        default_threads = torch.get_num_threads()
        try:
            threads = len(os.sched_getaffinity(0))
        except (AttributeError, OSError):
            threads = os.cpu_count() or default_threads
        torch.set_num_threads(threads)
        gen = torch.Generator().manual_seed(0)
        bf = torch.bfloat16

        # headline: SDPA fwd + bwd, bf16, the full configuration
        B, H, S, D = 1, 16, 1024, 128
        q, k, v, do = (torch.randn((B, H, S, D), generator=gen).to(bf) for _ in range(4))

        def aten():
            qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
            F.scaled_dot_product_attention(qq, kk, vv).backward(do)

        f, b = attn_flops(B, H, S, S, D)
        t_aten, n_aten = median_time(aten, self.args.cpu_seconds * 0.5)
        torch.set_num_threads(default_threads)
        t_def, n_def = median_time(aten, self.args.cpu_seconds * 0.1)
        torch.set_num_threads(threads)

        # the oracle port on 2 heads (float64 numpy)
        Hs = 2
        qa, ka, va, ga = (t[:, :Hs].double().numpy() for t in (q, k, v, do))
        sc = 1.0 / np.sqrt(D)

        def port():
            out, lse = oracle.attention_fwd(qa, ka, va, sc)
            oracle.attention_bwd(qa, ka, va, ga, lse, oracle.attention_delta(out, ga), sc)

        fp, bp = attn_flops(B, Hs, S, S, D)
        t_port, n_port = median_time(port, self.args.cpu_seconds * 0.1, at_least=3)

        # the other benchmark configurations
        budget = self.args.cpu_seconds * 0.3 / 7
        cfg = {}

        def rate(name, fn, work, unit, sample):
            t, n = median_time(fn, budget)
            scale = 1e12 if unit == "TFLOP/s" else 1e9
            cfg[name] = {"value": round(work / t / scale, 3), "unit": unit, "ms": round(t * 1e3, 3),
                         "sample": f"{sample}, median of {n} runs"}

        A, Bm, bias = (torch.randn(s_, generator=gen).to(bf) for s_ in ((1024, 1024), (1024, 1024), (1024,)))
        rate("addmm_1024_bias_bf16", lambda: torch.addmm(bias, A, Bm), 2.0 * 1024 ** 3, "TFLOP/s",
             "torch.addmm(bias[1024], A[1024,1024], B[1024,1024]) bf16")
        X, W = torch.randn((1024, 2048), generator=gen).to(bf), torch.randn((8192, 2048), generator=gen).to(bf)
        rate("mm_1024x2048x8192_nt_bf16", lambda: X @ W.t(), 2.0 * 1024 * 2048 * 8192, "TFLOP/s",
             "X[1024,2048] @ W[8192,2048]^T bf16 (F.linear layout)")
        xs = torch.randn((16384, 1024), generator=gen) * 2
        ys = torch.softmax(xs, -1)
        gs = torch.randn((16384, 1024), generator=gen)
        n4 = 16384 * 1024 * 4
        rate("softmax_fwd_f32_16384x1024", lambda: torch._softmax(xs, -1, False), 2 * n4, "GB/s", "aten::_softmax fp32")
        rate("softmax_bwd_f32_16384x1024", lambda: torch._softmax_backward_data(gs, ys, -1, torch.float32), 3 * n4, "GB/s",
             "aten::_softmax_backward_data fp32")
        xl, gl = (torch.randn((1024, 2048), generator=gen).to(bf) for _ in range(2))
        wl, bl = (torch.randn((2048,), generator=gen).to(bf) for _ in range(2))
        _, ml, rl = torch.native_layer_norm(xl, [2048], wl, bl, 1e-5)
        R_, D_ = 1024, 2048
        rate("layer_norm_fwd_bf16_1024x2048", lambda: torch.native_layer_norm(xl, [2048], wl, bl, 1e-5),
             2 * R_ * D_ * 2 + 2 * D_ * 2 + 2 * R_ * 4, "GB/s", "aten::native_layer_norm bf16 with weight and bias")
        rate("layer_norm_bwd_bf16_1024x2048",
             lambda: torch.ops.aten.native_layer_norm_backward(gl, xl, [2048], ml, rl, wl, bl, [True, True, True]),
             3 * R_ * D_ * 2 + D_ * 2 + 2 * R_ * 4 + 2 * D_ * 2, "GB/s", "aten::native_layer_norm_backward bf16 (dx, dw, db)")
        qi = torch.randint(-127, 128, (8192, 2048), generator=gen, dtype=torch.int8)
        si = (torch.rand((8192, 32), generator=gen) * 0.019 + 0.001).to(bf)
        rate("dequant_int8_8192x2048_bf16", lambda: (qi.float() * si.float().repeat_interleave(64, 1)[:, :2048]).to(bf),
             8192 * 2048 + 8192 * 32 * 2 + 8192 * 2048 * 2, "GB/s",
             "the reference's CPU closed form (torch_vulkan/__init__.py:203-205)")
        torch.set_num_threads(default_threads)
        return {"value": round((f + b) / t_aten / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "reference",
                "ms_per_sample": round(t_aten * 1e3, 2), "cpu_model": model, "os_cpu_count": os.cpu_count(),
                "sample": f"torch {torch.__version__} CPU aten F.scaled_dot_product_attention forward + backward, bf16, "
                          f"the full [1,16,1024,128] configuration (the reference's CPU path), median of {n_aten} runs "
                          f"on {threads} threads (every core in this process's affinity set), {model}",
                "default_pool": {"threads": default_threads, "value": round((f + b) / t_def / 1e12, 5),
                                 "ms_per_sample": round(t_def * 1e3, 2),
                                 "sample": f"the same on torch's default pool, median of {n_def} runs"},
                "configs": cfg,
                "oracle_port": {"value": round((fp + bp) / t_port / 1e12, 5), "unit": "TFLOP/s",
                                "ms_per_sample": round(t_port * 1e3, 1),
                                "sample": f"oracle.attention_fwd + attention_delta + attention_bwd (numpy float64) on "
                                          f"2 of the 16 heads, median of {n_port} runs"}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (every box here has one "
              "GPU; attention shards over independent (batch, head) pairs with no exchange)", file=sys.stderr)
        sys.exit(2)
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    bench = Bench(args)
    if args.profile:
        bench.profile(args.profile, args.steps)
        return
    print(f"[bench] device: {bench.tv.device_name()}", file=sys.stderr, flush=True)
    ms, tflops, kstats, roof = bench.attn_headline()
    print(f"[bench] attention fwd+bwd step {ms:.4f} ms = {tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)
    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) inputs, resident in HBM)",
        "config": {"workload": "flash-attention fwd+bwd, B=1 H=16 S=1024 D=128 bf16, non-causal, scale 1/sqrt(128) "
                               "(benchmark configs[1]+[2]); one step = F.scaled_dot_product_attention forward + "
                               "backward through autograd on the vk device ([B,S,H,D] tensors viewed via "
                               "transpose(1,2), as the reference's tools/bench_attention.py), which queues the fwd, "
                               "dQ (+delta) and dK/dV kernels",
                   "B": 1, "H": 16, "S": 1024, "D": 128, "parallelism": "single GPU"},
        "frac_of_bf16_peak": round(tflops / PEAK_BF16_TFLOPS, 4),
        "roofline": roof,
        "attn_kernels": kstats,
        "ms_per_step_gpu_events": round(bench.op_gpu_ms, 5),
        "kernel_step_ms": round(bench.kernel_step_ms, 5),
        "kernel_step_tflops": round(3.006477e10 / (bench.kernel_step_ms * 1e-3) / 1e12, 2),
        "ms_sum_of_kernel_averages": round(bench.kernel_sum_ms, 5),
        "attn_step_memory": bench.op_mem,
    }
    if not args.only_attn:
        line["attn_s4096"] = bench.attn_s4096()
        line["gemm"] = [bench.gemm(1024, 2048, 8192, "nt"), bench.gemm(1024, 2048, 8192, "nn"),
                        bench.gemm(1024, 1024, 1024, "nn", bias=True)]
        print(f"[bench] gemm {line['gemm']}", file=sys.stderr, flush=True)
        line["dq8_linear"] = [bench.dq8_linear(1024), bench.dq8_linear(4096)]
        line["dit_lora_stack"] = bench.dit_lora_stack()
        print(f"[bench] DiT LoRA stack {line['dit_lora_stack']}", file=sys.stderr, flush=True)
        line["dit_block"] = bench.dit_block()
        print(f"[bench] DiT block {line['dit_block']}", file=sys.stderr, flush=True)
        line["softmax_f32_16384x1024"] = bench.softmax()
        line["layer_norm_bf16_1024x2048"] = bench.layer_norm()
        line["dequant_int8_8192x2048_bf16"] = bench.dequant()
        line["elementwise"] = bench.elementwise()
        line["reductions"] = bench.reductions()
        line["block_swap_transfers"] = bench.transfers()
        line["image_ops"] = bench.image_ops()
        print("[bench] bandwidth kernels done", file=sys.stderr, flush=True)
    if not args.skip_cpu:
        line["cpu_baseline"] = bench.cpu_baseline()
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Benchmark of the gated-mixture Linear on one MI355X.

Workload (the headline shape): one gated Linear 5120 -> 17408 over 8192 tokens
with K = 6 candidates (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0).  A step is the
forward (mix W_eff + Y = X W_eff^T) and the backward (dX = dY W_eff and the
gate gradients <dY^T X, W_k>), called through the C ABI with every input
already resident in HBM.  value = 6*M*N*D / step time (TFLOP/s).

Also reported in the same JSON line:
  roofline      the dominant launch's achieved TFLOP/s against the bf16 MFMA
                peak (HIP events on the stream the kernels run on); the backward
                runs dX and the gate product in one launch
  kernels_ms    per-kernel average durations
  hipblaslt_ms  torch's bf16 matmul (hipBLASLt) on the same plain products
                (Y = X W_eff^T, dX = dY W_eff), for scale
  recipe_menu   the same step with the reference's 27B recipe menu (Q8_0,
                Q5_K, IQ3_S, IQ2_S, IQ2_XXS, IQ1_S): the IQ decode paths
  dequant_gbps  dequant microbench (4096 x 14336, each of the 14 formats):
                algorithmic bytes (packed read + fp32 write) / time, against
                8 TB/s
  cpu_baseline  the oracle's fp32 torch restatement of the reference step on
                the host cores, on a row sample of the same layer
  peaks         the chip's sustained bf16 MFMA rate (random and constant
                operands) and HBM read / copy / write bandwidth, measured by
                probe kernels (libvq_probe.so) in the same run; the roofline
                is also stated against the random-operand MFMA rate
  ptqr          the routed (per-token candidate) forward at the headline shape,
                and the bf16 decode of the six candidates it reads
  cpu_extra     the single-Linear configuration (512 tokens x 1024 -> 1024,
                K = 4) on the host (median of 5) and on the GPU, and the C
                dequant restatement per format, single- and multi-threaded
  host          nproc, the CPU model and sockets of the box
  shapes        mix, forward GEMM and backward launch times of the 27B-class
                layer's four products (q, o, gate/up, down) and the 0.8B-class
                decoder's four stacked products, 8192 tokens, K = 6
  fused         the few-token products with W_eff built in LDS (never in
                memory) against mix + GEMM, forward + dX, at 1-64 tokens on
                three tensor sizes: the measured crossover behind the module's
                choice of path
  attention     the decoder step's causal attention (batch 4, 16 heads, 2048
                positions, head dim 64): the HIP forward and backward against
                torch's memory-efficient SDPA kernels, us and TFLOP/s
  train         the 0.8B-class decoder gate-training step (4 x 2048 tokens,
                every Linear and the embedding gated, Q8_0 teacher): tokens/s,
                and the step time with torch's SDPA attention in its place
  stress        the 8-block SwiGLU stack at hidden 4096, MLP 14336, K = 8,
                2 x 8192 tokens: tokens/s
  stream_schedule  that stack with its candidates in pinned host memory:
                resident, copied in stream order, and copied ahead of use

  python bench.py --fused-workload runs only that comparison's kernels at 16
  tokens (three passes each), the workload the rocprof HBM-traffic summary of
  the fused kernels is taken on; --shapes-workload runs only the shape sweep;
  --attention-workload only the attention comparison.

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "voodoo-dyn-quant_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "gated-Linear fwd+bwd TFLOP/s + dequant HBM GB/s (% roofline); train tokens/sec"
TYPES = ["Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]
IQ_TYPES = ["IQ1_S", "IQ1_M", "IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S", "IQ4_XS"]
# the reference's 27B recipe menu (configs/qwen38_27b_voodoo30_tp4.sh:90)
RECIPE_TYPES = ["Q8_0", "Q5_K", "IQ3_S", "IQ2_S", "IQ2_XXS", "IQ1_S"]
GGML = {"Q8_0": 8, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ2_XXS": 16, "IQ2_XS": 17,
        "IQ3_XXS": 18, "IQ1_S": 19, "IQ3_S": 21, "IQ2_S": 22, "IQ4_XS": 23, "IQ1_M": 29}
BLOCK = {"Q8_0": (32, 34), "Q2_K": (256, 84), "Q3_K": (256, 110), "Q4_K": (256, 144), "Q5_K": (256, 176),
         "Q6_K": (256, 210), "IQ1_S": (256, 50), "IQ1_M": (256, 56), "IQ2_XXS": (256, 66), "IQ2_XS": (256, 74),
         "IQ2_S": (256, 82), "IQ3_XXS": (256, 98), "IQ3_S": (256, 110), "IQ4_XS": (256, 136)}
# fp16 scale fields (IQ1_M: none, its scale is spread over the top nibbles of bytes 49, 51, 53, 55)
F16_OFFSETS = {"Q8_0": (0,), "Q2_K": (80, 82), "Q3_K": (108,), "Q4_K": (0, 2), "Q5_K": (0, 2), "Q6_K": (208,),
               "IQ1_S": (0,), "IQ1_M": (), "IQ2_XXS": (0,), "IQ2_XS": (0,), "IQ2_S": (0,), "IQ3_XXS": (0,),
               "IQ3_S": (0,), "IQ4_XS": (0,)}
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBPS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synthetic_qbytes(torch, qt: str, nrows: int, ncols: int, dev, gen):
    """Random valid GGUF blocks generated on the device: random payload bytes,
    fp16 scale fields drawn from normal numbers in [2^-8, 2)."""
    bs, bb = BLOCK[qt]
    nblocks = nrows * ncols // bs
    q = torch.randint(0, 256, (nblocks, bb), dtype=torch.uint8, device=dev, generator=gen)
    for off in F16_OFFSETS[qt] or (None,):
        h = torch.randint(0, 1 << 16, (nblocks,), dtype=torch.int32, device=dev, generator=gen)
        h = (h & 0x83FF) | (0x1C00 + ((h >> 10) & 0x7) * 0x0400)  # exponent 7..14
        if off is None:  # IQ1_M: nibble t of the scale tops byte 49 + 2 t
            for t in range(4):
                q[:, 49 + 2 * t] = ((q[:, 49 + 2 * t].to(torch.int32) & 0x0F) | (((h >> (4 * t)) & 0xF) << 4)).to(torch.uint8)
            continue
        q[:, off] = (h & 0xFF).to(torch.uint8)
        q[:, off + 1] = ((h >> 8) & 0xFF).to(torch.uint8)
    return q.reshape(-1)


def time_events(torch, fn, reps: int, passes: int = 1) -> float:
    """Average milliseconds of fn() over reps, HIP events on the current
    stream; with passes > 1 the best pass (the first calls of a kernel on
    fresh buffers run while the clock and caches settle)."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(passes):
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        best = min(best, s.elapsed_time(e) / reps)
    return best


def host_info() -> dict:
    """Core count, CPU model and sockets of the host running the bench."""
    import platform
    import subprocess

    info = {"nproc": os.cpu_count(), "cpu_share_threads": int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or None}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Socket(s)", "Thread(s) per core", "Core(s) per socket"):
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        info["Model name"] = platform.processor()
    return info


def measured_peaks(torch, dev) -> dict:
    """Sustained bf16 MFMA rate (a long register-only stream of
    v_mfma_f32_32x32x16_bf16 on every SIMD, about 0.3 s, so the clock settles
    where the power limit puts it) and HBM bandwidth (a 4 GiB read, a
    2 GiB -> 2 GiB copy, a 4 GiB write), timed with HIP events on the launch
    stream.""" 
    import ctypes

    lib = ctypes.CDLL(str(ROOT / "voodoo-dyn-quant_amd" / "voodoo_quant" / "libvq_probe.so"))
    lib.vq_probe_mfma.argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    lib.vq_probe_hbm_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    lib.vq_probe_hbm_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    stream = torch.cuda.current_stream(dev).cuda_stream
    blocks = lib.vq_probe_mfma_blocks()
    sink = torch.empty(blocks * 256, dtype=torch.float32, device=dev)

    def mfma(iters):
        rc = lib.vq_probe_mfma(iters, sink.data_ptr(), stream)
        if rc:
            raise RuntimeError(f"vq_probe_mfma: hip error {rc}")

    t = time_events(torch, lambda: mfma(20000), 1)
    iters = max(20000, int(20000 * 300.0 / max(t, 1e-3)))
    t = time_events(torch, lambda: mfma(iters), 2)
    flop = blocks * 4.0 * iters * 8 * 32768
    rec = {"mfma_bf16_TFLOPs": round(flop / (t * 1e-3) / 1e12, 1), "mfma_probe_ms": round(t, 2)}
    # the same stream with a clock reading, on constant and on random operands
    # (the matrix pipe's power, hence the clock the card holds, follows how
    # many operand bits toggle; GEMMs on real data see random operands)
    lib.vq_probe_mfma_clock.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_uint32, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p]
    clocks = torch.zeros(2, dtype=torch.int64, device=dev)
    wall_khz = lib.vq_probe_wall_clock_khz() or 100000
    for name, rnd in (("const", 0), ("random", 1)):
        def run():
            rc = lib.vq_probe_mfma_clock(rnd, iters, 12345, sink.data_ptr(), clocks.data_ptr(), stream)
            if rc:
                raise RuntimeError(f"vq_probe_mfma_clock: hip error {rc}")
        t = time_events(torch, run, 2)
        ticks, rt = (int(v) for v in clocks.cpu())
        rec[f"mfma_bf16_{name}_TFLOPs"] = round(flop / (t * 1e-3) / 1e12, 1)
        # shader-clock ticks over real seconds (s_memrealtime ticks at the
        # runtime's constant wall-clock rate) over the same loop of block 0
        rec[f"mfma_{name}_clock_GHz"] = round(ticks / (rt / (wall_khz * 1e3)) / 1e9, 3) if rt > 0 else None
    hb = lib.vq_probe_hbm_blocks()
    hsink = torch.empty(hb * 256, dtype=torch.int32, device=dev)
    nbytes = 4 << 30
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    t = time_events(torch, lambda: lib.vq_probe_hbm_read(buf.data_ptr(), nbytes, hsink.data_ptr(), stream), 5)
    rec["hbm_read_GBps"] = round(nbytes / (t * 1e-3) / 1e9, 1)
    half = nbytes // 2
    t = time_events(torch, lambda: lib.vq_probe_hbm_copy(buf.data_ptr(), buf.data_ptr() + half, half, stream), 5)
    rec["hbm_copy_GBps"] = round(2 * half / (t * 1e-3) / 1e9, 1)
    lib.vq_probe_hbm_write.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    t = time_events(torch, lambda: lib.vq_probe_hbm_write(buf.data_ptr(), nbytes, stream), 5)
    rec["hbm_write_GBps"] = round(nbytes / (t * 1e-3) / 1e9, 1)
    del buf
    torch.cuda.empty_cache()
    log(f"measured peaks: {rec}")
    return rec


def _random_blocks_np(np, qt: str, nrows: int, ncols: int, rng):
    """Random valid blocks: random payload, fp16 scales with exponent 7..14."""
    bs, bb = BLOCK[qt]
    qb = rng.integers(0, 256, size=(nrows * ncols // bs, bb), dtype=np.uint8)
    for off in F16_OFFSETS[qt]:
        qb[:, off + 1] = (qb[:, off + 1] & 0x83) | (0x1C + (rng.integers(0, 8, size=qb.shape[0], dtype=np.uint8) << 2))
    return qb


def cpu_extra(torch, dev) -> dict:
    """The single-Linear configuration (1024 -> 1024, 512 tokens, K = 4:
    Q8_0, Q6_K, Q4_K, Q3_K; T = 1) as the oracle's fp32 torch step on the host
    (median of 5 after one warm-up) and as the HIP step on the GPU; and the C
    dequant restatement on the host per format, one thread and all threads
    (a 512 x 14336 row sample of the 4096 x 14336 microbench tensor)."""
    import numpy as np

    from oracle import cdequant, mixture
    from voodoo_quant import _hip

    types = ["Q8_0", "Q6_K", "Q4_K", "Q3_K"]
    m, n, d = 512, 1024, 1024
    rng = np.random.default_rng(1)
    g = torch.Generator().manual_seed(1)
    qbs = [_random_blocks_np(np, qt, n, d, rng) for qt in types]
    cands = [torch.from_numpy(cdequant.oracle_dequant(qt, qb, n * d).reshape(n, d)) for qt, qb in zip(types, qbs)]
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    gates = torch.randn(len(types), generator=g)
    mixture.reference_step_fp32(x, dy, cands, gates, 1.0)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        mixture.reference_step_fp32(x, dy, cands, gates, 1.0)
        times.append(time.perf_counter() - t0)
    cpu_ms = sorted(times)[2] * 1e3
    flops = mixture.gated_linear_flops(m, n, d)
    # the same step on the GPU (forward with W_eff, backward with dX and dL/dp)
    ids = [GGML[t] for t in types]
    qd = [torch.from_numpy(q.reshape(-1)).to(dev) for q in qbs]
    xd, dyd = x.to(dev), dy.to(dev)
    probs = torch.softmax(gates, 0).to(dev)
    w_eff = torch.empty(n, d, dtype=torch.bfloat16, device=dev)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    dx = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    dp = torch.empty(len(types), dtype=torch.float32, device=dev)
    ws = torch.empty(_hip.bwd_workspace_bytes(m, n, d, d, len(types), False), dtype=torch.uint8, device=dev)

    def step():
        _hip.gated_linear_fwd(xd, ids, qd, probs, n, d, w_eff, y)
        _hip.gated_linear_bwd(dyd, xd, ids, qd, probs, n, d, w_eff, dx, dp, ws)

    gpu_ms = time_events(torch, step, 50)
    rec = {"config1_1024x1024_m512_k4": {
        "cpu_ms": round(cpu_ms, 3), "cpu_TFLOPs": round(flops / (cpu_ms * 1e-3) / 1e12, 4),
        "gpu_ms": round(gpu_ms, 4), "gpu_TFLOPs": round(flops / (gpu_ms * 1e-3) / 1e12, 2),
        "cpu_threads": torch.get_num_threads(),
        "sample": "oracle fp32 torch step (mix + F.linear + autograd + <dW, W_k>), median of 5"}}
    dq = {}
    rows, cols = 512, 14336
    nthreads = torch.get_num_threads()
    for qt in TYPES:
        qb = _random_blocks_np(np, qt, rows, cols, rng)
        nbytes = qb.size + 4 * rows * cols
        r = {}
        for label, fn in (("1_thread", lambda: cdequant.oracle_dequant(qt, qb, rows * cols)),
                          (f"{nthreads}_threads",
                           lambda: cdequant.oracle_dequant_parallel(qt, qb, rows * cols, nthreads))):
            fn()
            t0 = time.perf_counter()
            fn()
            r[label + "_GBps"] = round(nbytes / (time.perf_counter() - t0) / 1e9, 2)
        dq[qt] = r
    rec["dequant_c_restatement"] = dq
    rec["dequant_sample"] = f"{rows} x {cols} rows of random valid blocks per format; bytes = packed read + fp32 write"
    log(f"cpu extra: config 1 cpu {cpu_ms:.1f} ms, gpu {gpu_ms:.3f} ms; dequant C {dq}")
    return rec


FUSED_SHAPES = [(1024, 3072), (4096, 4096), (5120, 17408)]  # (in_features, out_features)


def fused_compare(torch, dev, gen, tokens=(1, 16, 32, 64), reps: int = 20, passes: int = 0) -> dict:
    """Forward + dX of one gated Linear (K = 6) at a few tokens: the fused
    kernels (W_eff built tile by tile in LDS) against mix + GEMM (W_eff written
    to HBM, read by both GEMMs), in microseconds.  passes > 0 only runs each
    path that many times at 16 tokens (the profiling workload)."""
    from voodoo_quant import _hip

    ids = [GGML[t] for t in TYPES]
    out = {}
    for d, n in FUSED_SHAPES:
        qb = [synthetic_qbytes(torch, t, n, d, dev, gen) for t in TYPES]
        probs = torch.softmax(torch.randn(len(TYPES), device=dev, generator=gen), 0)
        w = torch.empty(n, d, dtype=torch.bfloat16, device=dev)
        rows = {}
        for m in ((16,) if passes else tokens):
            x = torch.randn(m, d, device=dev, generator=gen).to(torch.bfloat16)
            dy = torch.randn(m, n, device=dev, generator=gen).to(torch.bfloat16)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            dx = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
            wsf = torch.empty(max(_hip.fused_workspace_bytes(m, n, d, False), 16), dtype=torch.uint8, device=dev)
            wsd = torch.empty(max(_hip.fused_workspace_bytes(m, n, d, True), 16), dtype=torch.uint8, device=dev)
            # the materialised path with the workspaces the module passes (K-split
            # parts of the last tiles: at a few tokens the products have few tiles)
            wmf = torch.empty(max(_hip.fwd_workspace_bytes(m, n, d), 16), dtype=torch.uint8, device=dev)
            wmb = torch.empty(max(_hip.bwd_workspace_bytes(m, n, d, d, len(ids), False), 16), dtype=torch.uint8,
                              device=dev)

            def fused():
                _hip.gated_linear_fwd_fused(x, ids, qb, probs, n, d, y, wsf)
                _hip.gated_linear_dx_fused(dy, ids, qb, probs, d, d, dx, wsd)

            def materialised():
                _hip.gated_linear_fwd(x, ids, qb, probs, n, d, w, y, wmf)
                _hip.gated_linear_bwd(dy, x, ids, qb, probs, n, d, w, dx, None, wmb)

            if passes:
                for fn in (fused, materialised):
                    for _ in range(passes):
                        fn()
                    torch.cuda.synchronize()
                continue
            rows[m] = {"fused_us": round(time_events(torch, fused, reps) * 1e3, 1),
                       "materialised_us": round(time_events(torch, materialised, reps) * 1e3, 1)}
        out[f"{n}x{d}"] = rows
        del qb, w
        torch.cuda.empty_cache()
    if not passes:
        log(f"fused vs materialised (fwd + dX, us): {out}")
    return out


# Gated Linears timed by shape_sweep, M = 8192 tokens, K = 6 (Q2_K..Q8_0):
# the 27B-class layer's four products (hidden 5120, q/o 5120 x 6144, gate/up
# 5120 -> 17408, down 17408 -> 5120) and the 0.8B-class decoder's four stacked
# products (hidden 1024: q/k/v 1024 -> 1536, o 1024 -> 1024, gate/up
# 1024 -> 6144, down 3072 -> 1024), as (name, in_features, out_features).
SWEEP_SHAPES = [("27b_q", 5120, 6144), ("27b_o", 6144, 5120), ("27b_gate_up", 5120, 17408),
                ("27b_down", 17408, 5120), ("0p8b_qkv", 1024, 1536), ("0p8b_o", 1024, 1024),
                ("0p8b_gate_up", 1024, 6144), ("0p8b_down", 3072, 1024)]


def shape_sweep(torch, dev, gen, m: int = 8192, reps: int = 5) -> dict:
    """Per shape: the mix, the forward GEMM (``vq_linear_fwd`` over the
    premixed W_eff, timed on its own: at 1024-wide shapes the mix is a
    launch-latency-bound ~10-25 us that a difference of two timings would
    mostly measure) and the backward launch (dX + gate products, plus the gate
    reduce), HIP events on the stream the C ABI uses, with their TFLOP/s
    (2 m n d per product)."""
    from voodoo_quant import _hip

    ids = [GGML[t] for t in TYPES]
    res = {}
    for name, d, n in SWEEP_SHAPES:
        qbytes = [synthetic_qbytes(torch, qt, n, d, dev, gen) for qt in TYPES]
        x = torch.randn(m, d, device=dev, generator=gen).to(torch.bfloat16)
        dy = torch.randn(m, n, device=dev, generator=gen).to(torch.bfloat16)
        probs = torch.softmax(torch.randn(len(TYPES), device=dev, generator=gen), 0)
        w_eff = torch.empty(n, d, dtype=torch.bfloat16, device=dev)
        y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        dx = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
        dp = torch.empty(len(TYPES), dtype=torch.float32, device=dev)
        ws = torch.empty(_hip.bwd_workspace_bytes(m, n, d, d, len(TYPES), False), dtype=torch.uint8, device=dev)
        fws = torch.empty(max(_hip.fwd_workspace_bytes(m, n, d), 256), dtype=torch.uint8, device=dev)
        t_mix = time_events(torch, lambda: _hip.mix_weight(ids, qbytes, probs, n, d, w_eff), reps)
        t_gemm = time_events(torch, lambda: _hip.linear_fwd(x, w_eff, n, y, fws), reps)
        t_fwd = time_events(torch, lambda: _hip.gated_linear_fwd(x, ids, qbytes, probs, n, d, w_eff, y, fws), reps)
        t_bwd = time_events(torch, lambda: _hip.gated_linear_bwd(dy, x, ids, qbytes, probs, n, d, w_eff, dx, dp, ws),
                            reps)
        f = 2.0 * m * n * d
        res[name] = {"in": d, "out": n, "mix_ms": round(t_mix, 4), "fwd_gemm_ms": round(t_gemm, 4),
                     "fwd_ms": round(t_fwd, 4), "bwd_dx_gate_ms": round(t_bwd, 4),
                     "fwd_TFLOPs": round(f / (t_gemm * 1e-3) / 1e12, 1),
                     "bwd_TFLOPs": round(2 * f / (t_bwd * 1e-3) / 1e12, 1),
                     "step_TFLOPs": round(3 * f / ((t_fwd + t_bwd) * 1e-3) / 1e12, 1)}
        log(f"shape {name} {d}->{n}: mix {t_mix:.3f} ms, fwd gemm {t_gemm:.3f} ms (mix + gemm {t_fwd:.3f}), "
            f"bwd {t_bwd:.3f} ms")
        del qbytes, x, dy, w_eff, y, dx, ws, fws
    return res


def copy_calibration(torch, dev) -> None:
    """Three elementwise copies of 1 GiB (known bytes: 1 GiB read, 1 GiB
    written each), to scale rocprof's FETCH_SIZE / WRITE_SIZE."""
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    log("copy calibration: 3 x 1 GiB elementwise copy kernels")
    del src, dst


def cpu_baseline(torch, m: int, n_total: int, d: int, budget_s: float = 12.0) -> dict:
    """The reference step on the host: oracle fp32 torch restatement of
    _MixedWeightFunction + F.linear + autograd backward (voodoo_quant/
    layers.py:336-363), on rows [0, n_s) of the layer with all m tokens."""
    import numpy as np

    from oracle import cdequant, mixture

    n_s = 256
    g = torch.Generator().manual_seed(0)
    rng = np.random.default_rng(0)
    cands = []
    for qt in TYPES:
        bs, bb = BLOCK[qt]
        qb = rng.integers(0, 256, size=(n_s * d // bs, bb), dtype=np.uint16).astype(np.uint8)
        for off in F16_OFFSETS[qt]:
            h = rng.integers(0, 1 << 16, size=qb.shape[0]).astype(np.uint16)
            h = (h & 0x83FF) | (np.uint16(0x1C00) + ((h >> 10) & 0x7) * np.uint16(0x0400))
            qb[:, off], qb[:, off + 1] = (h & 0xFF).astype(np.uint8), (h >> 8).astype(np.uint8)
        cands.append(torch.from_numpy(cdequant.oracle_dequant_parallel(qt, qb, n_s * d).reshape(n_s, d)))
    x = torch.randn(m, d, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n_s, generator=g).to(torch.bfloat16)
    gates = torch.randn(len(TYPES), generator=g)
    mixture.reference_step_fp32(x, dy, cands, gates, 1.0)  # warm-up
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < 2:
        t0 = time.perf_counter()
        mixture.reference_step_fp32(x, dy, cands, gates, 1.0)
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    t = sorted(times)[len(times) // 2]
    flops = mixture.gated_linear_flops(m, n_s, d)
    return {
        "value": round(flops / t / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle fp32 torch step on rows 0..{n_s - 1} of the 5120->17408 layer (all {m} tokens, K=6), "
                  f"median of {len(times)} steps, {t * 1e3:.1f} ms/step; per-row work is the same as the full layer",
    }


def attention_bench(torch, dev, reps: int = 20) -> dict:
    """The decoder step's causal attention at its shape (batch 4, 16 heads,
    2048 positions, head dim 64, q/k/v/dO as [B, H, S, D] views of [B, S, H, D]
    memory, as the rotary kernel leaves them): vq_attention_fwd / _bwd against
    torch's memory-efficient SDPA forward and its backward kernel (run over the
    same forward's output and log-sum-exp).  FLOPs: forward 4 B H S^2 D / 2
    (causal), backward 2.5 x that (five products, S recomputed)."""
    import math

    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from voodoo_quant import _hip

    B, H, S, D = 4, 16, 2048, 64
    gen = torch.Generator(device=dev).manual_seed(3)
    q, k, v, do = (torch.randn(B, S, H, D, device=dev, generator=gen).to(torch.bfloat16).transpose(1, 2)
                   for _ in range(4))
    out, lse = _hip.attention_fwd(q, k, v)
    zero = torch.zeros((), dtype=torch.int64)
    scale = 1.0 / math.sqrt(D)

    def torch_fwd():
        with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, is_causal=True)

    def torch_bwd():
        return torch.ops.aten._scaled_dot_product_efficient_attention_backward(
            do, q, k, v, None, out, lse, zero, zero, 0.0, [True, True, True, False], True, scale=scale)

    t = {"fwd": time_events(torch, lambda: _hip.attention_fwd(q, k, v), reps, 2),
         "bwd": time_events(torch, lambda: _hip.attention_bwd(do, q, k, v, out, lse), reps, 2),
         "torch_fwd": time_events(torch, torch_fwd, reps, 2),
         "torch_bwd": time_events(torch, torch_bwd, reps, 2)}
    fwd_fl = 4.0 * B * H * S * S * D / 2
    fl = {"fwd": fwd_fl, "bwd": 2.5 * fwd_fl, "torch_fwd": fwd_fl, "torch_bwd": 2.5 * fwd_fl}
    rec = {"workload": "causal attention, batch 4, 16 heads, 2048 positions, head dim 64, bf16"}
    for key, ms in t.items():
        rec[f"{key}_us"] = round(ms * 1e3, 1)
        rec[f"{key}_TFLOPs"] = round(fl[key] / (ms * 1e-3) / 1e12, 1)
    rec["fwd_frac_of_spec"] = round(rec["fwd_TFLOPs"] / PEAK_BF16_TFLOPS, 3)
    rec["bwd_frac_of_spec"] = round(rec["bwd_TFLOPs"] / PEAK_BF16_TFLOPS, 3)
    log("attention us: " + ", ".join(f"{k} {v * 1e3:.1f}" for k, v in t.items()))
    return rec


def train_step_bench(torch, dev, steps: int, warmup: int, prefetch: bool = False, defer: bool = False) -> dict:
    """Gate-training steps of the 0.8B-class decoder (24 layers, hidden 1024,
    16x64 query heads, 4 KV heads, SwiGLU 3072, vocabulary 151936 tied; every
    Linear and the embedding gated over 6 candidates; Q8_0 teacher), batch
    4 x 2048 uniform-random token ids: tokens per second of the whole step
    (forwards, CE + KL + size loss, backward, clip, AdamW).  The teacher's
    forward runs on a second stream beside the student's; the plain GEMMs
    (teacher projections, heads) use the TunableOp results of
    step.use_tuned_gemms."""
    from voodoo_quant.training import step as st

    cfg = st.DecoderConfig()
    t0 = time.perf_counter()
    student, teacher, replaced = st.build_models(cfg, TYPES, dev, seed=0, packed=True)
    torch.cuda.synchronize()
    log(f"train: decoder built in {time.perf_counter() - t0:.1f} s ({len(replaced)} gated tensors)")
    b, s = 4, 2048
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randint(0, cfg.vocab, (b, s), device=dev, generator=g)
    y = torch.randint(0, cfg.vocab, (b, s), device=dev, generator=g)
    tr = st.GateTrainer(student, teacher, replaced,
                        st.StepConfig(max_steps=max(steps + warmup, 2), prefetch_mix=prefetch,
                                      teacher_stream=True, defer_gate_grads=defer, tuned_gemms=True),
                        total_8bit_bytes=float(cfg.gated_weights()))
    for _ in range(warmup):
        tr.step(x, y)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = tr.step(x, y)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / max(steps, 1) * 1e3
    from voodoo_quant import layers

    # the same step with torch's SDPA attention (AOTriton forward, its fused
    # backward) in place of the HIP attention kernels, for comparison
    saved = st.HIP_ATTENTION
    try:
        st.HIP_ATTENTION = False
        tr.step(x, y)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            tr.step(x, y)
        torch.cuda.synchronize()
        ms_sdpa = (time.perf_counter() - t0) / max(steps, 1) * 1e3
    finally:
        st.HIP_ATTENTION = saved
    layers.raise_pending_id_errors()  # the last step's deferred embedding id checks
    tokens = b * s
    fl = st.step_flops(cfg, tokens, s)
    rec = {"tokens_per_s": round(tokens / (ms * 1e-3), 1), "ms_per_step": round(ms, 3),
           "ms_per_step_torch_attention": round(ms_sdpa, 3), "steps": steps, "tuned_gemms": tr.tuned_gemms,
           "warmup": warmup, "model_TFLOPs": round(fl / (ms * 1e-3) / 1e12, 1),
           "loss": {k: round(float(v), 4) for k, v in out.items()},
           "workload": "0.8B-class decoder gate-training step: 24 layers, hidden 1024, 16x64 q heads, 4 KV heads, "
                       "SwiGLU 3072, vocab 151936 tied; 168 gated Linears + gated embedding, K=6; Q8_0 teacher; "
                       "batch 4x2048 uniform-random ids; CE + KL + dead-zone size loss at 45% of 8-bit",
           "candidate_bytes": "random valid GGUF blocks, scales sized for N(0, 0.02)-like weights"}
    log(f"train: {ms:.1f} ms/step -> {rec['tokens_per_s']:.0f} tokens/s ({rec['model_TFLOPs']} model TFLOP/s); "
        f"{ms_sdpa:.1f} ms/step with torch's attention")
    del student, teacher, replaced, tr
    torch.cuda.empty_cache()
    return rec


def stack_step_bench(torch, dev, steps: int, warmup: int, prefetch: bool = False, defer: bool = False) -> dict:
    """The long-context, wide-menu stress configuration: 8 SwiGLU blocks at
    hidden 4096, MLP 14336 (MLP-only blocks), K = 8 distinct formats per
    tensor (the six K-quant and Q8_0 formats plus IQ2_XXS and IQ3_S, two of the
    reference's 27B recipe types), 2 x 8192 tokens, temperature annealed
    2.0 -> 0.1 over 200 steps; tokens per second of the whole step (student,
    Q8_0 teacher, MSE + size loss, backward, optimizer)."""
    from voodoo_quant.training import step as st

    cfg = st.StackConfig()
    types = ["Q2_K", "IQ2_XXS", "Q3_K", "IQ3_S", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]
    student, teacher, replaced = st.build_stack(cfg, types, dev, seed=1)
    tokens = 2 * 8192
    g = torch.Generator(device=dev).manual_seed(6)
    x = torch.randn(tokens, cfg.hidden, device=dev, generator=g).to(torch.bfloat16)
    tr = st.StackTrainer(student, teacher, replaced,
                         st.StepConfig(max_steps=200, temp_start=2.0, temp_end=0.1, prefetch_mix=prefetch,
                                       defer_gate_grads=defer),
                         total_8bit_bytes=float(cfg.gated_weights()))
    for _ in range(warmup):
        tr.step(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = tr.step(x)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / max(steps, 1) * 1e3
    fl = st.stack_flops(cfg, tokens)
    rec = {"tokens_per_s": round(tokens / (ms * 1e-3), 1), "ms_per_step": round(ms, 3), "steps": steps,
           "warmup": warmup, "model_TFLOPs": round(fl / (ms * 1e-3) / 1e12, 1),
           "loss": {k: round(float(v), 5) for k, v in out.items()},
           "workload": "8 SwiGLU blocks (MLP-only) at hidden 4096, MLP 14336: 24 gated tensors, 1.409e9 weights, "
                       "K=8 (Q2_K, IQ2_XXS, Q3_K, IQ3_S, Q4_K, Q5_K, Q6_K, Q8_0); 2 x 8192 tokens; "
                       "T 2.0 -> 0.1 over 200 steps; "
                       "relative MSE to a Q8_0 teacher + dead-zone size loss at 45% of 8-bit",
           "candidate_bytes": "random valid GGUF blocks, scales sized for N(0, 0.02)-like weights"}
    log(f"stack: {ms:.1f} ms/step -> {rec['tokens_per_s']:.0f} tokens/s ({rec['model_TFLOPs']} model TFLOP/s)")
    del student, teacher, replaced, tr, x
    torch.cuda.empty_cache()
    return rec


def stream_schedule_bench(torch, dev, steps: int = 3, warmup: int = 2, slots: int = 6, depth: int = 5) -> dict:
    """The stress step with its candidates in pinned host memory instead of
    HBM (a model whose candidates do not fit on the GPU): every product's
    packed bytes are copied host -> device before its forward and again
    before its backward, as the reference does every step
    (``layers.py:348, 362``).  Timed three ways on one model: candidates
    resident (no copies), streamed in stream order (each copy in front of its
    product, the reference's pattern), and streamed ahead of use on a copy
    stream (``streaming.CandidateStreamer``, `depth` products ahead through
    `slots` device slots).  Also the host -> device rate of one 1 GiB pinned
    copy."""
    from voodoo_quant.training import step as st

    cfg = st.StackConfig()
    types = ["Q2_K", "IQ2_XXS", "Q3_K", "IQ3_S", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]
    student, teacher, replaced = st.build_stack(cfg, types, dev, seed=1)
    tokens = 2 * 8192
    g = torch.Generator(device=dev).manual_seed(6)
    x = torch.randn(tokens, cfg.hidden, device=dev, generator=g).to(torch.bfloat16)
    cand_bytes = sum(q.numel() for m in replaced.values() for q in m._qbytes())

    def timed(**stream):
        tr = st.StackTrainer(student, teacher, replaced,
                             st.StepConfig(max_steps=200, temp_start=2.0, temp_end=0.1, **stream),
                             total_8bit_bytes=float(cfg.gated_weights()))
        for _ in range(warmup):
            tr.step(x)
        torch.cuda.synchronize()
        copied0 = tr.streamer.bytes_copied if tr.streamer else 0
        t0 = time.perf_counter()
        for _ in range(steps):
            tr.step(x)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / max(steps, 1) * 1e3
        copied = ((tr.streamer.bytes_copied - copied0) / max(steps, 1)) if tr.streamer else 0
        if tr.streamer:
            tr.streamer.release()
        tr.bank.release()
        return ms, copied

    def timeline():
        """One overlapped step with the streamer's timing events: when the copy
        engine is busy, by phase (forward, the turn between the last forward
        fence and the first backward fence, backward)."""
        tr = st.StackTrainer(student, teacher, replaced,
                             st.StepConfig(max_steps=200, temp_start=2.0, temp_end=0.1, stream_candidates=True,
                                           stream_slots=slots, stream_depth=depth, stream_timeline=True),
                             total_8bit_bytes=float(cfg.gated_weights()))
        for _ in range(warmup):
            tr.step(x)
        torch.cuda.synchronize()
        tr.streamer.timeline.clear()
        origin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        origin.record()
        tr.step(x)
        end.record()
        torch.cuda.synchronize()
        events = tr.streamer.timeline_ms(origin)
        step_ms = origin.elapsed_time(end)
        tr.streamer.release()
        tr.bank.release()
        copies = sorted((a, b) for kind, _, a, b in events if kind == "copy")
        fwd_end = max((a for kind, _, a, _ in events if kind == "forward"), default=0.0)
        bwd_start = min((a for kind, _, a, _ in events if kind == "backward"), default=step_ms)

        def busy(lo, hi):  # copy-engine time inside [lo, hi]
            total, cur = 0.0, lo
            for a, b in copies:
                a, b = max(a, cur), min(b, hi)
                if b > a:
                    total += b - a
                    cur = b
            return total

        phases = {"forward": (0.0, fwd_end), "turn": (fwd_end, bwd_start), "backward": (bwd_start, step_ms)}
        out = {"step_ms": round(step_ms, 2), "copies": len(copies),
               "copy_busy_ms": round(busy(0.0, step_ms), 2)}
        for name, (lo, hi) in phases.items():
            out[f"{name}_ms"] = round(hi - lo, 2)
            out[f"{name}_copy_busy_frac"] = round(busy(lo, hi) / (hi - lo), 3) if hi > lo else None
        return out

    resident_ms, _ = timed()
    serial_ms, serial_bytes = timed(stream_candidates=True, stream_overlap=False, stream_slots=slots,
                                    stream_depth=depth)
    overlap_ms, overlap_bytes = timed(stream_candidates=True, stream_slots=slots, stream_depth=depth)
    tl = timeline()
    host = torch.empty(1 << 30, dtype=torch.uint8, pin_memory=True)
    devbuf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    t = time_events(torch, lambda: devbuf.copy_(host, non_blocking=True), 3)
    h2d = (1 << 30) / (t * 1e-3) / 1e9
    rec = {"resident_ms": round(resident_ms, 2), "streamed_serial_ms": round(serial_ms, 2),
           "streamed_overlap_ms": round(overlap_ms, 2),
           "overlap_speedup_vs_serial": round(serial_ms / overlap_ms, 3),
           "candidate_bytes": cand_bytes, "copied_bytes_per_step_serial": int(serial_bytes),
           "copied_bytes_per_step_overlap": int(overlap_bytes), "h2d_GBps": round(h2d, 1),
           "copy_floor_ms": round(overlap_bytes / (h2d * 1e9) * 1e3, 2), "slots": slots, "depth": depth,
           "overlap_timeline": tl,
           "workload": "the stress step (8 SwiGLU blocks, hidden 4096, MLP 14336, K=8, 2 x 8192 tokens) with "
                       "its 24 tensors' candidates in pinned host memory, copied before each forward and backward"}
    log(f"stream schedule: resident {resident_ms:.1f} ms, streamed in order {serial_ms:.1f} ms, overlapped "
        f"{overlap_ms:.1f} ms (copies {overlap_bytes / 1e9:.2f} GB/step at {h2d:.1f} GB/s)")
    log(f"stream schedule timeline (one overlapped step): {tl}")
    del student, teacher, replaced, x, host, devbuf
    torch.cuda.empty_cache()
    return rec


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-train", action="store_true", help="skip the decoder gate-training step measurement")
    ap.add_argument("--train-steps", type=int, default=5)
    ap.add_argument("--only-train", action="store_true",
                    help="measure only the decoder gate-training step and print its record")
    ap.add_argument("--no-stack", action="store_true", help="skip the 8-block SwiGLU stress measurement")
    ap.add_argument("--no-stream", action="store_true",
                    help="skip the stress step with candidates streamed from host memory")
    ap.add_argument("--only-stream", action="store_true",
                    help="measure only the stress step with streamed candidates and print its record")
    ap.add_argument("--only-stack", action="store_true",
                    help="measure only the 8-block SwiGLU stress step and print its record")
    ap.add_argument("--prefetch-mix", action="store_true",
                    help="train/stress steps mix each W_eff ahead on a second stream (layers.MixPrefetch)")
    ap.add_argument("--defer-gate-grads", action="store_true",
                    help="train/stress steps finish the gate gradients on a second stream (trainer.GateBank)")
    ap.add_argument("--no-peaks", action="store_true", help="skip the MFMA / HBM probe kernels")
    ap.add_argument("--no-sweeps", action="store_true",
                    help="skip the per-shape and few-token sweeps (profiles of the headline shape alone)")
    ap.add_argument("--fused-workload", action="store_true",
                    help="only run the fused and materialising few-token products (16 tokens, 3 passes each)")
    ap.add_argument("--shapes-workload", action="store_true",
                    help="only time the 27B-class and 0.8B-class gated Linear shapes and print their record")
    ap.add_argument("--attention-workload", action="store_true",
                    help="only time the decoder step's attention forward and backward (HIP and torch) and print them")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device copy (known bytes) to scale rocprof FETCH/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the gated Linear's multi-GPU sharding is a design note, not a run)", file=sys.stderr)
        return 2

    import torch

    from voodoo_quant import _hip

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.fused_workload:
        fused_compare(torch, dev, torch.Generator(device=dev).manual_seed(0), passes=3)
        if args.copy_calibration:
            copy_calibration(torch, dev)
        return 0
    if args.shapes_workload:
        print(json.dumps({"shapes": shape_sweep(torch, dev, torch.Generator(device=dev).manual_seed(0))}),
              flush=True)
        return 0
    if args.attention_workload:
        print(json.dumps({"attention": attention_bench(torch, dev)}), flush=True)
        return 0
    if args.only_train:
        print(json.dumps({"train": train_step_bench(torch, dev, args.train_steps, 2, args.prefetch_mix, args.defer_gate_grads)}), flush=True)
        return 0
    if args.only_stream:
        print(json.dumps({"stream_schedule": stream_schedule_bench(torch, dev)}), flush=True)
        return 0
    if args.only_stack:
        print(json.dumps({"stress": stack_step_bench(torch, dev, 3, 2, args.prefetch_mix, args.defer_gate_grads)}), flush=True)
        return 0
    m, n, d = 8192, 17408, 5120
    d_pad = d
    ids = [GGML[t] for t in TYPES]
    gen = torch.Generator(device=dev).manual_seed(0)
    log(f"building synthetic candidates {TYPES} for {n}x{d}")
    qbytes = [synthetic_qbytes(torch, qt, n, d_pad, dev, gen) for qt in TYPES]
    x = torch.randn(m, d, device=dev, generator=gen).to(torch.bfloat16)
    dy = torch.randn(m, n, device=dev, generator=gen).to(torch.bfloat16)
    probs = torch.softmax(torch.randn(len(TYPES), device=dev, generator=gen), 0)
    w_eff = torch.empty(n, d_pad, dtype=torch.bfloat16, device=dev)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    dx = torch.empty(m, d, dtype=torch.bfloat16, device=dev)
    dp = torch.empty(len(TYPES), dtype=torch.float32, device=dev)
    ws = torch.empty(_hip.bwd_workspace_bytes(m, n, d, d_pad, len(TYPES), False), dtype=torch.uint8, device=dev)
    fws = torch.empty(max(_hip.fwd_workspace_bytes(m, n, d), 256), dtype=torch.uint8, device=dev)

    def fwd():
        _hip.gated_linear_fwd(x, ids, qbytes, probs, n, d_pad, w_eff, y, fws)

    def bwd():
        _hip.gated_linear_bwd(dy, x, ids, qbytes, probs, n, d_pad, w_eff, dx, dp, ws)

    def step():
        fwd()
        bwd()

    log(f"warmup {args.warmup} steps")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) / max(args.steps, 1) * 1e3
    flops = 6.0 * m * n * d
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"step {ms:.3f} ms -> {tflops:.1f} TFLOP/s")

    # per-kernel durations (HIP events on torch's current stream, which the C ABI uses)
    reps = 5
    t_mix = time_events(torch, lambda: _hip.mix_weight(ids, qbytes, probs, n, d_pad, w_eff), reps)
    t_fwd = time_events(torch, fwd, reps)
    t_dx = time_events(torch, lambda: _hip.gated_linear_bwd(dy, x, ids, qbytes, probs, n, d_pad, w_eff, dx, None,
                                                            ws), reps)
    t_gate = time_events(torch, lambda: _hip.gated_linear_bwd(dy, x, ids, qbytes, probs, n, d_pad, w_eff, None, dp,
                                                              ws), reps)
    t_bwd = time_events(torch, bwd, reps)
    gemm_flops = 2.0 * m * n * d
    # bwd_dx_gate: the backward's single launch of both products (plus the
    # few-microsecond gate reduce); dx_gemm / gate_gemm: each product alone
    kernels = {"mix_w_eff": t_mix, "fwd_gemm": t_fwd - t_mix, "bwd_dx_gate": t_bwd, "dx_gemm": t_dx,
               "gate_gemm": t_gate}
    launch_flops = {"fwd_gemm": gemm_flops, "bwd_dx_gate": 2 * gemm_flops}
    dom = max(launch_flops, key=lambda k: kernels[k])
    achieved = launch_flops[dom] / (kernels[dom] * 1e-3) / 1e12
    traffic = None
    tfile = ROOT / "profiles" / "traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get(dom)
    log("kernels ms: " + ", ".join(f"{k} {v:.3f}" for k, v in kernels.items()))

    # the same step with the reference's 27B recipe menu (four IQ formats): the
    # IQ instantiations of the mix, gate epilogue and dual backward
    iq_ids = [GGML[t] for t in RECIPE_TYPES]
    iq_q = [synthetic_qbytes(torch, qt, n, d_pad, dev, gen) for qt in RECIPE_TYPES]
    iq_probs = torch.softmax(torch.randn(len(RECIPE_TYPES), device=dev, generator=gen), 0)

    def iq_fwd():
        _hip.gated_linear_fwd(x, iq_ids, iq_q, iq_probs, n, d_pad, w_eff, y, fws)

    def iq_bwd():
        _hip.gated_linear_bwd(dy, x, iq_ids, iq_q, iq_probs, n, d_pad, w_eff, dx, dp, ws)

    t_iq_step = time_events(torch, lambda: (iq_fwd(), iq_bwd()), reps)
    t_iq_mix = time_events(torch, lambda: _hip.mix_weight(iq_ids, iq_q, iq_probs, n, d_pad, w_eff), reps)
    t_iq_bwd = time_events(torch, iq_bwd, reps)
    iq_menu = {"candidates": RECIPE_TYPES, "step_ms": round(t_iq_step, 4),
               "TFLOPs": round(flops / (t_iq_step * 1e-3) / 1e12, 1), "mix_w_eff_ms": round(t_iq_mix, 4),
               "bwd_dx_gate_ms": round(t_iq_bwd, 4),
               "candidate_bytes": sum(int(q.numel()) for q in iq_q)}
    del iq_q
    log(f"recipe menu {RECIPE_TYPES}: step {t_iq_step:.3f} ms, mix {t_iq_mix:.3f} ms, bwd {t_iq_bwd:.3f} ms")
    # the vendor library on the same plain products, for scale: torch's bf16
    # matmul (hipBLASLt) for Y = X W_eff^T and dX = dY W_eff
    w_c = w_eff[:, :d].contiguous()
    for _ in range(2):  # hipBLASLt's first calls at a shape run slower
        torch.nn.functional.linear(x, w_c)
        torch.matmul(dy, w_c)
    lib = {"fwd_gemm": time_events(torch, lambda: torch.nn.functional.linear(x, w_c), 2 * reps),
           "dx_gemm": time_events(torch, lambda: torch.matmul(dy, w_c), 2 * reps)}
    del w_c
    log("hipBLASLt ms (same shapes, plain bf16 products): " + ", ".join(f"{k} {v:.3f}" for k, v in lib.items()))

    # PTQR routed forward at the same shape: tokens Gumbel-routed from probs,
    # one grouped GEMM over the cached bf16 candidate decodes
    from voodoo_quant import layers

    cand_bf16 = [_hip.dequant_bf16(GGML[qt], qb, n, d_pad) for qt, qb in zip(TYPES, qbytes)]
    t_dec = time_events(torch, lambda: [_hip.dequant_bf16(GGML[qt], qb, n, d_pad, c)
                                        for qt, qb, c in zip(TYPES, qbytes, cand_bf16)], 3)
    routing = layers._sample_token_routing(probs, m)
    perm = torch.argsort(routing, stable=True).to(torch.int32)
    goff = torch.zeros(len(TYPES) + 1, dtype=torch.int32, device=dev)
    goff[1:] = torch.cumsum(torch.bincount(routing, minlength=len(TYPES)), 0).to(torch.int32)
    t_routed = time_events(torch, lambda: _hip.routed_linear_fwd(x, cand_bf16, perm, goff, n, d_pad, y), 10, 3)
    ptqr = {"routed_fwd_ms": round(t_routed, 4), "routed_fwd_TFLOPs": round(gemm_flops / (t_routed * 1e-3) / 1e12, 1),
            "bf16_decode_all_candidates_ms": round(t_dec, 4)}
    del cand_bf16
    log(f"ptqr: routed fwd {t_routed:.3f} ms, bf16 decode of {len(TYPES)} candidates {t_dec:.3f} ms")

    # dequant microbench, 4096 x 14336
    dq = {}
    nr, nc = 4096, 14336
    out = torch.empty(nr, nc, dtype=torch.float32, device=dev)
    for qt in TYPES + IQ_TYPES:
        qb = synthetic_qbytes(torch, qt, nr, nc, dev, gen)
        t = time_events(torch, lambda: _hip.dequant(GGML[qt], qb, nr, nc, out), 10)
        nbytes = qb.numel() + 4 * nr * nc
        dq[qt] = {"GBps": round(nbytes / (t * 1e-3) / 1e9, 1), "ms": round(t, 4),
                  "frac": round(nbytes / (t * 1e-3) / 1e9 / PEAK_HBM_GBPS, 3)}
        del qb
    log("dequant GB/s: " + ", ".join(f"{k} {v['GBps']}" for k, v in dq.items()))

    del qbytes, w_eff, y, dx, ws, fws, out
    torch.cuda.empty_cache()
    shapes = None if args.no_sweeps else shape_sweep(torch, dev, gen)
    attention = None if args.no_sweeps else attention_bench(torch, dev)
    train = None
    if not args.no_train:
        torch.cuda.empty_cache()
        train = train_step_bench(torch, dev, args.train_steps, 2, args.prefetch_mix, args.defer_gate_grads)
    stack = None
    if not args.no_stack:
        stack = stack_step_bench(torch, dev, 3, 2, args.prefetch_mix, args.defer_gate_grads)
    stream = None
    if not args.no_stream and not args.no_stack:
        stream = stream_schedule_bench(torch, dev)

    if args.copy_calibration:
        copy_calibration(torch, dev)

    peaks = None if args.no_peaks else measured_peaks(torch, dev)
    fused = None if args.no_sweeps else fused_compare(torch, dev, gen)

    cpu = extra = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(torch, m, n, d)
        extra = cpu_extra(torch, dev)

    rec = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "gated Linear fwd+bwd, 8192 tokens x 5120->17408, K=6 candidates",
            "tokens": m, "in_features": d, "out_features": n, "candidates": TYPES,
            "candidate_bytes": "random valid GGUF blocks (no libggml on the box)",
        },
        "roofline": {
            "kernel": dom, "bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
            # the sustained rate of an MFMA stream on random operands (what a
            # GEMM on real data can draw at the card's power limit); the
            # constant-operand stream's rate is in "peaks"
            "peak_measured": peaks["mfma_bf16_random_TFLOPs"] if peaks else None,
            "frac_of_measured": round(achieved / peaks["mfma_bf16_random_TFLOPs"], 4) if peaks else None,
        },
        "peaks": peaks,
        "fused": fused,
        "kernels_ms": {k: round(v, 4) for k, v in kernels.items()},
        "recipe_menu": iq_menu,
        "hipblaslt_ms": {k: round(v, 4) for k, v in lib.items()},
        "dequant_gbps": dq,
        "ptqr": ptqr,
        "shapes": shapes,
        "attention": attention,
        "train": train,
        "stress": stack,
        "stream_schedule": stream,
        "cpu_baseline": cpu,
        "cpu_extra": extra,
        "host": host_info(),
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

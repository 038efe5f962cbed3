#!/usr/bin/env python3
"""Benchmark of the CrossDiT attention node on one MI355X.

A step is one pass of the hot path -- rope::apply on Q and K followed by
the GGML_OP_FLASH_ATTN_EXT node -- at the production self-attention shape:
Q/K/V bf16 [128, 31744, 32, 2] (512x512, 121 frames -> latent 31x64x64,
patch (1,2,2) -> 31x32x32 tokens, CFG batch 2), 3-D RoPE (axes 32/48/48,
theta 1e4, scale factor (1,2,2)), scale 1/sqrt(128), no mask, F32 output,
through kd_fa_rope_run_ws: K rotated once into a K-sized workspace (the
buffer the unfused graph casts the rotated K into), Q rotated on load.
Inputs are synthetic N(0,1) from a fixed seed and already resident in HBM.

Prints ONE JSON line with the metric, the roofline of the attention kernel
and a CPU baseline (the oracle's restatement of ggml's CPU algorithm on a
bounded row sample, rank 0 only).  Secondary figures (the single-kernel
kd_fa_rope_run, the 1,280- and 62,464-token self-attention, the text
cross-attention, the VAE's D = 512 attention, the DiT linear layers through
kd_mm_run, the 60-layer step-equivalent) go in "secondary".
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kandinsky.cpp_amd"))

PEAK_BF16_TFLOPS = 2516.6      # 256 CU x 4096 flop/clk x 2.4 GHz, dense
PEAK_HBM_GBS = 8000.0
HEADS, D = 32, 128
AXES, SCALE_FACTOR, THETA = (32, 48, 48), (1.0, 2.0, 2.0), 10000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--rope", choices=["table", "axes"], default="table")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--cpu-rows", type=int, default=1024,
                   help="query rows per (b, h) in the CPU sample of the 31,744-token self-attention")
    p.add_argument("--cpu-rows-long", type=int, default=256,
                   help="query rows per head in the CPU sample of the 62,464-token self-attention")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only copy 1 GiB device-to-device 3 times (scales the PMC byte counters)")
    p.add_argument("--linear-only", action="store_true",
                   help="time only the 63,488 x 4096 x 4096 projection (BF16 weight rows, F32 x, bias) "
                        "and print its ms per call (for counter runs)")
    p.add_argument("--cross-only", action="store_true",
                   help="only the text cross-attention (C2 shape): for counter runs of its kernel")
    p.add_argument("--cross-long-only", action="store_true",
                   help="only the long-prompt cross-attention in the reference's operand form (Q F32 "
                        "[128, 31744, 32, 2], K/V F16 with 512 keys, no mask): for counter runs of its kernel")
    p.add_argument("--hbm-ceiling", action="store_true",
                   help="only torch's bf16 -> F32 copy at the cross-attention's sizes (its Q-in / O-out "
                        "byte mix) and a 1 GiB F32 copy")
    return p.parse_args()


def rand(torch, shape, seed, dev, dtype):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(dtype)


def traffic_from_profile():
    """HBM bytes per launch from the committed PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", "fa_fwd_c3_hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch:"):
                return float(line.split(":", 1)[1].split()[0])
    return None


def time_launches(torch, fn, steps, warmup, stream):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def cpu_share():
    """Host threads a one-GPU job may use: OMP_NUM_THREADS (the host's CPU
    share for one GPU), else the CPUs this process may run on."""
    try:
        n = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        n = 0
    return n if n > 0 else len(os.sched_getaffinity(0))


def cpu_baseline(torch, dev, q3, k3, v3, table3, rows3, rows4):
    """The oracle's restatement of ggml's per-row CPU flash-attention
    algorithm (ggml_compute_forward_flash_attn_ext_f16) on the host cores
    (rank 0, N=1 only): the 1,280-token self-attention and the text
    cross-attention in full, the 31,744- and 62,464-token self-attention on
    query-row samples (cost is linear in the rows at a fixed key count, so
    their full-call times are extrapolated).  The C3 rate is the reported
    value; it is a baseline, not the optimisation target."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import kd_oracle as orc

    threads = cpu_share()
    cfgs = {}

    def timed(q, k, v, mask=None, rope=None, rows=None):
        t0 = time.perf_counter()
        _, used = orc.fa_ggml(q, k, v, mask=mask, rope=rope, rows=rows, n_threads=threads)
        return time.perf_counter() - t0, used

    # C1: [128, 1280, 32, 1] f16, RoPE 5x16x16, every row
    L1 = 5 * 16 * 16
    q1, k1, v1 = (rand(torch, (1, HEADS, L1, D), 1 + 1000 * j, dev, torch.float16).cpu() for j in range(3))
    t1 = torch.from_numpy(orc.visual_rope_table(5, 16, 16, AXES, SCALE_FACTOR, THETA))
    dt, used = timed(q1, k1, v1, rope=orc.rope_table(t1))
    fl1 = 4.0 * HEADS * L1 * L1 * D
    cfgs["C1_1280_full"] = {"ms": round(dt * 1e3, 2), "tflops": round(fl1 / dt / 1e12, 4), "rows": HEADS * L1}
    # C2: Q [128, 31744, 32, 2] x K/V 256 bf16, padding mask 120 / 40, every row
    B, L = q3.shape[0], q3.shape[2]
    k2, v2 = (rand(torch, (B, HEADS, 256, D), 1002 + 1000 * j, dev, torch.bfloat16).cpu() for j in range(2))
    m2 = torch.full((B, 1, L, 256), float("-inf"), dtype=torch.float16)
    m2[0, :, :, :120] = 0
    m2[1, :, :, :40] = 0
    qc = q3.cpu()
    dt, _ = timed(qc, k2, v2, mask=m2)
    bytes2 = (qc.numel() + k2.numel() + v2.numel()) * 2 + m2.numel() * 2 + qc.numel() * 4
    cfgs["C2_cross_full"] = {"ms": round(dt * 1e3, 2), "GBps": round(bytes2 / dt / 1e9, 2), "rows": B * HEADS * L}
    del k2, v2, m2
    # C3: the benchmarked workload, rows3 query rows per (b, h)
    rng = np.random.default_rng(0)
    rows = np.concatenate([rng.choice(L, rows3, replace=False) + L * (h + HEADS * b)
                           for b in range(B) for h in range(HEADS)]).astype(np.int64)
    kc, vc = k3.cpu(), v3.cpu()
    dt3, used = timed(qc, kc, vc, rope=orc.rope_table(torch.from_numpy(table3)), rows=rows)
    fl3 = 4.0 * len(rows) * L * D
    c3 = fl3 / dt3 / 1e12
    cfgs["C3_31744_sample"] = {"ms_extrapolated": round(dt3 * 1e3 * L / rows3, 1), "tflops": round(c3, 4),
                               "rows": len(rows), "sample_s": round(dt3, 2)}
    del qc, kc, vc
    # C4: [128, 62464, 32, 1] bf16, RoPE 61x32x32, rows4 query rows per head
    L4 = 61 * 32 * 32
    q4, k4, v4 = (rand(torch, (1, HEADS, L4, D), 4 + 1000 * j, dev, torch.bfloat16).cpu() for j in range(3))
    t4 = torch.from_numpy(orc.visual_rope_table(61, 32, 32, AXES, SCALE_FACTOR, THETA))
    rows = np.concatenate([rng.choice(L4, rows4, replace=False) + L4 * h for h in range(HEADS)]).astype(np.int64)
    dt4, _ = timed(q4, k4, v4, rope=orc.rope_table(t4), rows=rows)
    fl4 = 4.0 * len(rows) * L4 * D
    cfgs["C4_62464_sample"] = {"ms_extrapolated": round(dt4 * 1e3 * L4 / rows4, 1),
                               "tflops": round(fl4 / dt4 / 1e12, 4), "rows": len(rows), "sample_s": round(dt4, 2)}
    del q4, k4, v4
    return {"value": round(c3, 6), "unit": "TFLOP/s", "cores": used, "host_cores": os.cpu_count(),
            "kind": "port",
            "sample": (f"ggml per-row CPU flash-attn algorithm (restated, oracle/kd_oracle.c; F16 V accumulator "
                       f"converted by F16C as ggml's SIMD path does) on {used} threads "
                       f"(the CPU share of a one-GPU job; {os.cpu_count()} cores on the host): value = the "
                       f"31,744-token self-attention with RoPE on {rows3} query rows per (b,h) x {B * HEADS} "
                       f"heads, all keys ({dt3:.2f} s wall); the 1,280-token self-attention and the text "
                       f"cross-attention timed in full, the 62,464-token one on {rows4} rows per head"),
            "configs": cfgs}


def rope_rows_f32(torch, x, c, s):
    """rope::apply on F32 rows x (..., 128) with per-row (cos, sin) halves c,
    s (..., 64): every product and sum rounded to F32 on its own."""
    x0, x1 = x[..., 0::2], x[..., 1::2]
    o0 = x0 * c - x1 * s
    o1 = x0 * s + x1 * c
    return torch.stack((o0, o1), dim=-1).flatten(-2)


def lazy_cap_steps(torch, q, k, table, cap, waves=16, seed=5):
    """How often the 64-row kernel's lazy row max leaves its fast path on
    these operands: for `waves` sampled waves (64 consecutive query rows of
    one (b, h)), the logits in the log2 domain from the rotated operands
    rounded to K's type, then the kernel's rule per row -- the running max is
    the first tile's exact max; a later 64-key tile whose weight sum
    exp2(s - m) leaves [0, cap] moves m to that tile's max -- and a wave's
    step is slow when any of its rows moves.  Returns the fraction of the
    steps after the first that are slow (a model, in float64 on the GPU)."""
    B, H, L, Dh = q.shape
    tab = torch.from_numpy(table).to(q.device)
    c, s = tab[:, 0::2], tab[:, 1::2]
    g = torch.Generator().manual_seed(seed)
    scale = math.log2(math.e) / math.sqrt(Dh)
    slow, total = 0, 0
    for _ in range(waves):
        b = int(torch.randint(0, B, (1,), generator=g))
        h = int(torch.randint(0, H, (1,), generator=g))
        r0 = int(torch.randint(0, L // 64, (1,), generator=g)) * 64
        kr = rope_rows_f32(torch, k[b, h].float(), c, s).to(k.dtype).double()
        qr = rope_rows_f32(torch, q[b, h, r0:r0 + 64].float(), c[r0:r0 + 64], s[r0:r0 + 64]).to(k.dtype).double()
        sc = (qr @ kr.T) * scale                              # (64, L) log2 domain
        n_t = (L + 63) // 64
        m = sc[:, :64].max(dim=1).values
        for t in range(1, n_t):
            st = sc[:, 64 * t:64 * t + 64]
            tot = torch.exp2(st - m[:, None]).sum(dim=1)
            move = ~(tot <= cap)
            if bool(move.any()):
                slow += 1
                m = torch.where(move, torch.maximum(m, st.max(dim=1).values), m)
            total += 1
    return round(slow / max(total, 1), 6)


def self_check(torch, q, k, v, table, out, scale, rows_per_head=4, seed=11):
    """Sampled rows of the last step's output against a float64 torch
    reference of the same op on the same operands (rope::apply in F32,
    rounded to the operand type, then textbook softmax attention), on the
    GPU: the parity gate max-abs <= 2e-2, cosine >= 0.9995."""
    B, H, L, Dh = q.shape
    tab = torch.from_numpy(table).to(q.device)
    c, s = tab[:, 0::2], tab[:, 1::2]
    g = torch.Generator().manual_seed(seed)
    worst, dot, n_got, n_ref = 0.0, 0.0, 0.0, 0.0
    for b in range(B):
        for h in range(H):
            idx = torch.randint(0, L, (rows_per_head,), generator=g).to(q.device)
            kr = rope_rows_f32(torch, k[b, h].float(), c, s).to(k.dtype).double()
            qr = rope_rows_f32(torch, q[b, h, idx].float(), c[idx], s[idx]).to(k.dtype).double()
            p = torch.softmax((qr @ kr.T) * scale, dim=-1)
            ref = p @ v[b, h].double()
            got = out[b, idx, h, :].double()
            worst = max(worst, float((got - ref).abs().max()))
            dot += float((got * ref).sum())
            n_got += float((got * got).sum())
            n_ref += float((ref * ref).sum())
    cos = dot / (n_got * n_ref) ** 0.5
    ok = worst <= 2e-2 and cos >= 0.9995 and math.isfinite(worst)
    return {"rows": B * H * rows_per_head, "max_abs": worst, "cos": round(cos, 8), "pass": ok,
            "reference": "torch float64 on the GPU, same rounded operands (not the oracle)"}


def hbm_ceiling(torch, dev, stream):
    """What this GPU sustains for the cross-attention's byte mix: torch's own
    copy of a bf16 array of the C2 query size (520 MB) into an F32 array
    (1.04 GB written), and a 1 GiB F32 device copy; the mean of 20 launches
    each (HIP events on the launch stream)."""
    n = 2 * HEADS * 31744 * D
    src = torch.ones(n, dtype=torch.bfloat16, device=dev)
    dst = torch.empty(n, dtype=torch.float32, device=dev)
    res = {"bytes_read": n * 2, "bytes_written": n * 4}
    ms = time_launches(torch, lambda: dst.copy_(src), 20, 3, stream)
    res["torch_copy_bf16_to_f32"] = {"GBps": round(n * 6 / (ms * 1e-3) / 1e9, 1), "ms": round(ms, 4),
                                     "frac_of_8TBps": round(n * 6 / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    a = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    ms = time_launches(torch, lambda: b.copy_(a), 20, 3, stream)
    res["torch_copy_f32_1GiB"] = {"GBps": round(2 * a.numel() * 4 / (ms * 1e-3) / 1e9, 1), "ms": round(ms, 4)}
    return res


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the attention node runs on a single MI355X "
              "(multi-GPU sharding is a design note, not implemented)", file=sys.stderr)
        sys.exit(2)

    import torch
    import kd_fa

    dev = "cuda:0"
    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)   # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel() * 4, "copies": 3}))
        return
    stream = torch.cuda.current_stream()
    if args.hbm_ceiling:
        print(json.dumps(hbm_ceiling(torch, dev, stream)), flush=True)
        return
    B, T, Hp, Wp = 2, 31, 32, 32
    L = T * Hp * Wp
    bf = torch.bfloat16
    if args.cross_only:
        qx = rand(torch, (B, HEADS, L, D), 3, dev, bf)
        kx = rand(torch, (B, HEADS, 256, D), 1002, dev, bf)
        vx = rand(torch, (B, HEADS, 256, D), 2002, dev, bf)
        mx = torch.full((B, 1, L, 256), float("-inf"), dtype=torch.float16, device=dev)
        mx[0, :, :, :120] = 0
        mx[1, :, :, :40] = 0
        ox = torch.empty((B, L, HEADS, D), device=dev, dtype=torch.float32)
        dx = kd_fa.make_desc(qx, kx, vx, mx, ox, 1.0 / D ** 0.5)
        wsx = torch.empty(max(kd_fa.workspace_size_full(dx), 16), dtype=torch.uint8, device=dev)
        msx = time_launches(torch, lambda: kd_fa.run_desc(dx, None, stream, wsx), args.steps, args.warmup, stream)
        print(json.dumps({"cross_attn_ms": round(msx, 4)}))
        return
    if args.cross_long_only:
        ql = rand(torch, (B, HEADS, L, D), 3, dev, torch.float32)
        kl = rand(torch, (B, HEADS, 512, D), 1612, dev, torch.float16)
        vl = rand(torch, (B, HEADS, 512, D), 2612, dev, torch.float16)
        ol = torch.empty((B, L, HEADS, D), device=dev, dtype=torch.float32)
        dlong = kd_fa.make_desc(ql, kl, vl, None, ol, 1.0 / D ** 0.5)
        msl = time_launches(torch, lambda: kd_fa.run_desc(dlong, None, stream), args.steps, args.warmup, stream)
        print(json.dumps({"cross_attn_long_512_ms": round(msl, 4)}))
        return
    if args.linear_only:
        import kd_mm
        Mx = B * L
        xl = rand(torch, (Mx, 4096), 51, dev, torch.float32)
        yl = torch.empty((Mx, 4096), device=dev, dtype=torch.float32)
        bl = rand(torch, (4096,), 52, dev, torch.float32)
        wl = rand(torch, (4096, 4096), 53, dev, bf) * 0.05
        dl = kd_mm.make_desc(wl, xl, bl, yl)
        st = kd_mm.run_desc(dl, None, stream)
        if st != 0:
            raise kd_fa.KdFaError(st, "kd_mm_run")
        msl = time_launches(torch, lambda: kd_mm.run_desc(dl, None, stream), args.steps, args.warmup, stream)
        print(json.dumps({"linear_ms": round(msl, 4), "tflops": round(2.0 * Mx * 4096 * 4096 / (msl * 1e-3) / 1e12, 2)}))
        return
    q = rand(torch, (B, HEADS, L, D), 3, dev, bf)
    k = rand(torch, (B, HEADS, L, D), 1003, dev, bf)
    v = rand(torch, (B, HEADS, L, D), 2003, dev, bf)
    out = torch.empty((B, L, HEADS, D), device=dev, dtype=torch.float32)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    if args.rope == "table":
        rope = kd_fa.rope_table(torch.from_numpy(table).to(dev))
    else:
        axes = kd_fa.axes_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
        rope = kd_fa.rope_axes(torch.from_numpy(axes).to(dev), (T, Hp, Wp), AXES)
    desc = kd_fa.make_desc(q, k, v, None, out, 1.0 / D ** 0.5)
    ws = torch.empty(k.numel(), dtype=k.dtype, device=dev)

    def step():
        st = kd_fa.run_desc(desc, rope, stream, ws)
        if st != 0:
            raise kd_fa.KdFaError(st, "kd_fa_rope_run_ws")

    torch.cuda.synchronize()
    ms = time_launches(torch, step, args.steps, args.warmup, stream)
    check = self_check(torch, q, k, v, table, out, 1.0 / D ** 0.5)
    flop = 4.0 * B * HEADS * L * L * D
    tflops = flop / (ms * 1e-3) / 1e12
    res = {
        "metric": "self-attn TFLOP/s & % bf16 MFMA peak, 31.7k-token CrossDiT layer; ms/step",
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
        "data": "synthetic N(0,1), seeded, resident in HBM",
        "config": {"workload": "CrossDiT visual self-attention, 512x512x121f: Q/K/V bf16 [128, 31744, 32, 2], "
                               f"3-D RoPE grid 31x32x32 ({args.rope}) + attention via kd_fa_rope_run_ws, "
                               "scale 1/sqrt(128), no mask, F32 out",
                   "global_batch": B, "seq_len": L, "heads": HEADS, "head_dim": D, "parallelism": "single GPU"},
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "parity_check": check,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profile(),
                     "traffic_source": "constant read from profiles/fa_fwd_c3_hbm_traffic.txt (rocprofv3 --pmc "
                                       "FETCH_SIZE and WRITE_SIZE of this kernel at this shape, scaled by the "
                                       "same counters on a 1 GiB device copy); not measured in this run",
                     "kernel": "kdfa::fa_fwd_w64<bf16, RoPE table on Q, K from workspace> (64 query rows "
                               "per wave); achieved is over the whole step, which also holds the K "
                               "rotation pass (rope_k_kernel, <1% of it)",
                     "flop_per_launch": flop},
    }

    if not args.no_secondary:
        sec = {}
        # the same pass without a workspace (kd_fa_rope_run): K rotated by the
        # pre-pass into output rows that a later head group overwrites, the
        # 64-row kernel group by group, the last group rotating K on load;
        # bitwise equal
        ms_f = time_launches(torch, lambda: kd_fa.run_desc(desc, rope, stream), args.steps, args.warmup, stream)
        sec["self_attn_fused_ms"] = round(ms_f, 4)
        sec["self_attn_fused_tflops"] = round(flop / (ms_f * 1e-3) / 1e12, 2)
        sec["self_attn_fused_note"] = ("kd_fa_rope_run, no workspace: K staged in output rows of later head "
                                       "groups, the last group rotating K on load")
        # the reference's own operand form of this node (ops.hpp:122-169 via
        # crossdit.hpp:150): Q F32, K/V F16 after ggml_cast, RoPE table, through
        # kd_fa_rope_run_ws; on N(0,1) data and with peaked logits (Q and K
        # scaled by 2: logit std 4), where the F16 sum cap (2^15) can send a
        # wave's step to the exact-max slow path
        for tag, sc in (("n01", 1.0), ("peaked_std4", 2.0)):
            qf = rand(torch, (B, HEADS, L, D), 3, dev, torch.float32) * sc
            kf = (rand(torch, (B, HEADS, L, D), 1003, dev, torch.float32) * sc).half()
            vf = rand(torch, (B, HEADS, L, D), 2003, dev, torch.float16)
            of = torch.empty((B, L, HEADS, D), device=dev, dtype=torch.float32)
            dfx = kd_fa.make_desc(qf, kf, vf, None, of, 1.0 / D ** 0.5)
            wsf = torch.empty(kd_fa.workspace_size(dfx), dtype=torch.uint8, device=dev)
            msf = time_launches(torch, lambda: kd_fa.run_desc(dfx, rope, stream, wsf), 5, 1, stream)
            sec[f"self_attn_refform_{tag}_ms"] = round(msf, 4)
            sec[f"self_attn_refform_{tag}_tflops"] = round(flop / (msf * 1e-3) / 1e12, 2)
            sec[f"self_attn_refform_{tag}_slow_steps"] = lazy_cap_steps(torch, qf, kf, table, 2.0 ** 15)
            del qf, kf, vf, of, wsf
        sec["self_attn_refform_note"] = ("Q F32 [128, 31744, 32, 2], K/V F16, RoPE table, kd_fa_rope_run_ws; "
                                         "slow_steps: a model of the 64-row kernel's lazy max on 16 sampled "
                                         "waves (64 rows x all keys each): fraction of 64-key steps after the "
                                         "first in which a row's weight sum leaves [0, 2^15]")
        # all three operands F32 (the node as ops::attention receives it,
        # before its ggml_cast of K and V to F16): the pre-pass rotates and
        # casts K and casts V into the workspace
        q32, k32, v32 = (rand(torch, (B, HEADS, L, D), s_, dev, torch.float32) for s_ in (3, 1003, 2003))
        o32 = torch.empty((B, L, HEADS, D), device=dev, dtype=torch.float32)
        d32 = kd_fa.make_desc(q32, k32, v32, None, o32, 1.0 / D ** 0.5)
        ws32 = torch.empty(kd_fa.workspace_size(d32), dtype=torch.uint8, device=dev)
        ms32 = time_launches(torch, lambda: kd_fa.run_desc(d32, rope, stream, ws32), 5, 1, stream)
        sec["self_attn_all_f32_ms"] = round(ms32, 4)
        sec["self_attn_all_f32_tflops"] = round(flop / (ms32 * 1e-3) / 1e12, 2)
        sec["self_attn_all_f32_note"] = ("Q/K/V F32 [128, 31744, 32, 2], RoPE table, kd_fa_rope_run_ws: one "
                                         "pre-pass rotates and casts K and casts V to F16, then the attention")
        del q32, k32, v32, o32, ws32
        # the attention alone on unrotated operands (kd_fa_run)
        ms_n = time_launches(torch, lambda: kd_fa.run_desc(desc, None, stream), args.steps, args.warmup, stream)
        sec["self_attn_norope_ms"] = round(ms_n, 4)
        sec["self_attn_norope_tflops"] = round(flop / (ms_n * 1e-3) / 1e12, 2)
        # the DiT attention from the projections on (kd_fa_dit_run): query/key
        # RMSNorm, RoPE, attention, K through the workspace
        wq = rand(torch, (D,), 7, dev, torch.float32) * 0.3 + 1.0
        wk = rand(torch, (D,), 8, dev, torch.float32) * 0.3 + 1.0
        norm = kd_fa.qk_norm(wq, wk, 1e-6)
        ms_d = time_launches(torch, lambda: kd_fa.run_desc(desc, rope, stream, ws, norm), args.steps, args.warmup,
                             stream)
        sec["self_attn_norm_rope_ws_ms"] = round(ms_d, 4)
        sec["self_attn_norm_rope_ws_tflops"] = round(flop / (ms_d * 1e-3) / 1e12, 2)
        # the other self-attention shapes, through the same kd_fa_rope_run_ws
        # path: 1,280 tokens (f16, RoPE grid 5x16x16, batch 1; launch-bound)
        # and 62,464 tokens (bf16, RoPE grid 61x32x32, batch 1)
        for tag, (Bx, Tx, dt, seed) in (("c1_1280", (1, 5, torch.float16, 1)), ("c4_62464", (1, 61, bf, 4))):
            Hx = 16 if tag.startswith("c1") else 32
            Lx = Tx * Hx * Hx
            qx = rand(torch, (Bx, HEADS, Lx, D), seed, dev, dt)
            kx = rand(torch, (Bx, HEADS, Lx, D), seed + 1000, dev, dt)
            vx = rand(torch, (Bx, HEADS, Lx, D), seed + 2000, dev, dt)
            ox = torch.empty((Bx, Lx, HEADS, D), device=dev, dtype=torch.float32)
            tx = kd_fa.visual_rope_table(Tx, Hx, Hx, AXES, SCALE_FACTOR, THETA)
            ropex = kd_fa.rope_table(torch.from_numpy(tx).to(dev))
            dx = kd_fa.make_desc(qx, kx, vx, None, ox, 1.0 / D ** 0.5)
            wsx = torch.empty(kx.numel(), dtype=kx.dtype, device=dev)
            n = 100 if tag.startswith("c1") else 3
            msx = time_launches(torch, lambda: kd_fa.run_desc(dx, ropex, stream, wsx), n, 3 if n > 3 else 1, stream)
            flx = 4.0 * Bx * HEADS * Lx * Lx * D
            sec[f"self_attn_{tag}_ms"] = round(msx, 4)
            sec[f"self_attn_{tag}_tflops"] = round(flx / (msx * 1e-3) / 1e12, 2)
            sec[f"self_attn_{tag}_pct_bf16_peak"] = round(100.0 * flx / (msx * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2)
            if tag.startswith("c1"):
                # kd_fa_rope_run without a workspace: one launch rotating K on load
                msy = time_launches(torch, lambda: kd_fa.run_desc(dx, ropex, stream), n, 3, stream)
                sec[f"self_attn_{tag}_no_ws_ms"] = round(msy, 4)
            del qx, kx, vx, ox, wsx
        # a token count that is not a multiple of 64: 768x432, 121 frames ->
        # latent 31 x 54 x 96, patch (1, 2, 2) -> 31 x 27 x 48 = 40,176 tokens,
        # batch 2, with and without the K workspace
        Tr, Hr, Wr = 31, 27, 48
        Lr = Tr * Hr * Wr
        qr, kr, vr = (rand(torch, (B, HEADS, Lr, D), 70 + j, dev, bf) for j in range(3))
        orr = torch.empty((B, Lr, HEADS, D), device=dev, dtype=torch.float32)
        ropr = kd_fa.rope_table(torch.from_numpy(kd_fa.visual_rope_table(Tr, Hr, Wr, AXES, SCALE_FACTOR, THETA)).to(dev))
        dr = kd_fa.make_desc(qr, kr, vr, None, orr, 1.0 / D ** 0.5)
        wsr = torch.empty(kr.numel(), dtype=bf, device=dev)
        flr = 4.0 * B * HEADS * Lr * Lr * D
        for tag, wsx in (("ws", wsr), ("staged", None)):
            msr = time_launches(torch, lambda: kd_fa.run_desc(dr, ropr, stream, wsx), 3, 1, stream)
            sec[f"self_attn_ragged_{Lr}_{tag}_ms"] = round(msr, 4)
            sec[f"self_attn_ragged_{Lr}_{tag}_tflops"] = round(flr / (msr * 1e-3) / 1e12, 2)
        del qr, kr, vr, orr, wsr
        # text cross-attention: Q 31,744 x K/V 256, batch 2, padding mask 120 / 40 valid keys
        k2 = rand(torch, (B, HEADS, 256, D), 1002, dev, bf)
        v2 = rand(torch, (B, HEADS, 256, D), 2002, dev, bf)
        m2 = torch.full((B, 1, L, 256), float("-inf"), dtype=torch.float16, device=dev)
        m2[0, :, :, :120] = 0
        m2[1, :, :, :40] = 0
        out2 = torch.empty((B, L, HEADS, D), device=dev, dtype=torch.float32)
        d2 = kd_fa.make_desc(q, k2, v2, m2, out2, 1.0 / D ** 0.5)
        # kd_fa_run_ws: the mask summary pass, then the short-key kernel,
        # which skips the fully masked key tiles of each 32-row block without
        # loading their mask rows; kd_fa_run (no workspace) beside it
        # (after the long self-attention runs above this GPU's clock recovers
        # over tens of milliseconds: the two forms are timed alternately,
        # twice each, and the second timing of each is reported)
        ws2m = torch.empty(max(kd_fa.workspace_size_full(d2), 16), dtype=torch.uint8, device=dev)
        for _ in range(2):
            ms2n = time_launches(torch, lambda: kd_fa.run_desc(d2, None, stream), 50, 10, stream)
            ms2 = time_launches(torch, lambda: kd_fa.run_desc(d2, None, stream, ws2m), 50, 10, stream)
        bytes2 = (q.numel() + k2.numel() + v2.numel()) * 2 + m2.numel() * 2 + out2.numel() * 4
        sec["cross_attn_ms"] = round(ms2, 4)
        sec["cross_attn_GBps"] = round(bytes2 / (ms2 * 1e-3) / 1e9, 1)
        sec["cross_attn_hbm_frac"] = round(bytes2 / (ms2 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
        sec["cross_attn_note"] = ("kd_fa_run_ws (mask summary in the workspace); "
                                  "the measured ceiling for this byte mix: bench.py --hbm-ceiling")
        sec["cross_attn_no_ws_ms"] = round(ms2n, 4)
        # the reference's own cross-attention operand form (ops.hpp:122-169,
        # crossdit.hpp:198): Q F32, K/V F16, no mask, prompt lengths 77, 300
        # and 512 (the longest after the tokenizer's crop)
        q32 = rand(torch, (B, HEADS, L, D), 3, dev, torch.float32)
        o32 = torch.empty((B, L, HEADS, D), device=dev, dtype=torch.float32)
        for Lk in (77, 300, 512):
            kf = rand(torch, (B, HEADS, Lk, D), 1100 + Lk, dev, torch.float16)
            vf = rand(torch, (B, HEADS, Lk, D), 2100 + Lk, dev, torch.float16)
            df = kd_fa.make_desc(q32, kf, vf, None, o32, 1.0 / D ** 0.5)
            msf = time_launches(torch, lambda: kd_fa.run_desc(df, None, stream), 20, 3, stream)
            bf_ = q32.numel() * 4 + (kf.numel() + vf.numel()) * 2 + o32.numel() * 4
            ff_ = 4.0 * B * HEADS * L * Lk * D
            sec[f"cross_attn_f16_unmasked_{Lk}_ms"] = round(msf, 4)
            sec[f"cross_attn_f16_unmasked_{Lk}_GBps"] = round(bf_ / (msf * 1e-3) / 1e9, 1)
            sec[f"cross_attn_f16_unmasked_{Lk}_tflops"] = round(ff_ / (msf * 1e-3) / 1e12, 1)
            del kf, vf
        del q32, o32
        # the same with query/key RMSNorm and O stored as bf16 for out_layer
        out2b = torch.empty((B, L, HEADS, D), device=dev, dtype=torch.bfloat16)
        d2b = kd_fa.make_desc(q, k2, v2, m2, out2b, 1.0 / D ** 0.5)
        ws2 = torch.empty(kd_fa.workspace_size_full(d2b, None, norm), dtype=torch.uint8, device=dev)
        ms2b = time_launches(torch, lambda: kd_fa.run_desc(d2b, None, stream, ws2, norm), 20, 3, stream)
        bytes2b = bytes2 - out2.numel() * 2
        sec["cross_attn_norm_bf16out_ms"] = round(ms2b, 4)
        sec["cross_attn_norm_bf16out_GBps"] = round(bytes2b / (ms2b * 1e-3) / 1e9, 1)
        # the 2-D VAE's attention block (one head, D = 512, Q F32, K/V F16)
        # at 64x64 and 128x128 latents (512- and 1024-pixel images)
        for L5 in (4096, 16384):
            q5 = rand(torch, (1, 1, L5, 512), 41, dev, torch.float32)
            k5 = rand(torch, (1, 1, L5, 512), 42, dev, torch.float16)
            v5 = rand(torch, (1, 1, L5, 512), 43, dev, torch.float16)
            o5 = torch.empty((1, L5, 1, 512), device=dev, dtype=torch.float32)
            d5 = kd_fa.make_desc(q5, k5, v5, None, o5, 512 ** -0.5)
            # kd_fa_run_ws: with fewer than 256 blocks of 32 query rows the
            # keys of every row are split into ranges merged through the
            # workspace (4,096 tokens: two); kd_fa_run beside it
            ws5 = torch.empty(max(kd_fa.workspace_size_full(d5), 16), dtype=torch.uint8, device=dev)
            ms5v = time_launches(torch, lambda: kd_fa.run_desc(d5, None, stream, ws5), 20, 10, stream)
            ms5n = time_launches(torch, lambda: kd_fa.run_desc(d5, None, stream), 20, 10, stream)
            sec[f"vae_attn_{L5}_ms"] = round(ms5v, 4)
            sec[f"vae_attn_{L5}_tflops"] = round(4.0 * L5 * L5 * 512 / (ms5v * 1e-3) / 1e12, 2)
            sec[f"vae_attn_{L5}_no_ws_ms"] = round(ms5n, 4)
            del q5, k5, v5, o5, ws5
        # the DiT linear layers (ops::linear) at 63,488 tokens (31,744 x CFG 2):
        # a 4096 x 4096 projection with Q8_0 weights expanded into the
        # workspace on every call, the same with the weights kept as BF16 rows
        # (F32 and BF16 activations), and the two feed-forward products
        import kd_mm
        Mx = B * L
        wq8 = kd_mm.QuantWeight(torch.randint(0, 256, (4096, 4096 // 32 * 34), dtype=torch.uint8, device=dev),
                                kd_mm.TYPE_Q8_0, 4096)
        wq8.blocks.view(4096, 128, 34)[:, :, 1] = 0x20      # F16 scales of moderate size
        for tag, (N_, K_, xdt, wkind) in (("qkv_q8_0_f32x", (4096, 4096, torch.float32, "q8")),
                                          ("qkv_bf16w_f32x", (4096, 4096, torch.float32, "bf16")),
                                          ("qkv_bf16w_bf16x", (4096, 4096, bf, "bf16")),
                                          ("ffn_up_bf16w_f32x", (16384, 4096, torch.float32, "bf16")),
                                          ("ffn_down_bf16w_f32x", (4096, 16384, torch.float32, "bf16"))):
            xl = rand(torch, (Mx, K_), 51, dev, xdt)
            yl = torch.empty((Mx, N_), device=dev, dtype=torch.float32)
            bl = rand(torch, (N_,), 52, dev, torch.float32)
            if wkind == "q8":
                wl = wq8
            else:
                wl = rand(torch, (N_, K_), 53, dev, bf) * 0.05
            dl = kd_mm.make_desc(wl, xl, bl, yl)
            wsl = torch.empty(max(kd_mm.workspace_size(dl), 16), dtype=torch.uint8, device=dev)
            msl = time_launches(torch, lambda: kd_mm.run_desc(dl, wsl, stream), 10, 2, stream)
            fll = 2.0 * Mx * N_ * K_
            sec[f"linear_{tag}_ms"] = round(msl, 4)
            sec[f"linear_{tag}_tflops"] = round(fll / (msl * 1e-3) / 1e12, 2)
            if tag == "qkv_bf16w_bf16x":
                # the library GEMM (hipBLASLt through torch) on the same BF16
                # operands, with the node's F32 output and with a BF16 one
                wt = wl.t()
                for otag, fn in (("f32out", lambda: torch.mm(xl, wt, out_dtype=torch.float32)),
                                 ("bf16out", lambda: torch.mm(xl, wt))):
                    try:
                        msh = time_launches(torch, fn, 10, 2, stream)
                    except (TypeError, RuntimeError) as exc:
                        sec[f"linear_{tag}_hipblaslt_{otag}_error"] = str(exc)[:120]
                        continue
                    sec[f"linear_{tag}_hipblaslt_{otag}_ms"] = round(msh, 4)
                    sec[f"linear_{tag}_hipblaslt_{otag}_tflops"] = round(fll / (msh * 1e-3) / 1e12, 2)
            del xl, yl, wl, dl, wsl
        # 60 x (self + cross) with fresh buffers per layer (3 rotating sets)
        sets = [(q, k, v)] + [tuple(rand(torch, (B, HEADS, L, D), 10 * s + j, dev, bf) for j in range(3))
                              for s in range(1, 3)]
        descs = []
        for (qq, kk, vv) in sets:
            descs.append((kd_fa.make_desc(qq, kk, vv, None, out, 1.0 / D ** 0.5),
                          kd_fa.make_desc(qq, k2, v2, m2, out2, 1.0 / D ** 0.5)))

        def layer_stack():
            for i in range(60):
                ds, dc = descs[i % 3]
                kd_fa.run_desc(ds, rope, stream, ws)
                kd_fa.run_desc(dc, None, stream, ws2m)

        ms5 = time_launches(torch, layer_stack, 2, 1, stream)
        sec["step_equivalent_ms"] = round(ms5, 2)
        sec["step_equivalent_note"] = ("60 x (self-attn via kd_fa_rope_run_ws + cross-attn via kd_fa_run_ws), "
                                       "batch 2 CFG, 3 rotating input sets")
        res["secondary"] = sec
        del sets, descs

    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(torch, dev, q, k, v, table, args.cpu_rows, args.cpu_rows_long)
    print(json.dumps(res), flush=True)
    if not check["pass"]:
        print(f"bench.py: the output failed its parity check: {check}", file=sys.stderr)
        sys.exit(3)


if __name__ == "__main__":
    main()

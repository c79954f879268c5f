#!/usr/bin/env python3
"""Benchmark of the routed-expert path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--extras]

Headline (one JSON line on stdout): int4 expert decode mat-vec HBM GB/s.
A step is one token's 384 routed-expert evaluations at the Qwen3-30B-A3B
expert shape (48 layers x top-8; H=2048, I=768, int4 group 32, f16 scales) in
one fused layer call (gate|up, SiLU, down, weighted sum), the experts drawn
from a resident pool of 1024 (2.7 GB, beyond the 256 MB MALL) so every step
streams its 1.02 GB of packed weights from HBM. Inputs are resident before the
timed region. The value is algorithmic bytes (packed nibbles + f16 scales of
each expert touched once, plus activations) per second over the timed steps.

roofline: the dominant kernel (the int4 decode mat-vec, gate|up and down
launches) timed with HIP events on the launch stream inside the timed region.
cpu_baseline: the C/OpenMP restatement of the reference's numba kernel
(oracle/cpuref.c, _moe_q4 loop structure) on the host cores, a bounded sample.

roofline.traffic: HBM bytes per launch of that kernel, read from the counter
summary committed beside the kernel-trace summary
(profiles/mv_fast_kernel_int4_decode_384experts.md: rocprofv3 FETCH_SIZE and
WRITE_SIZE per dispatch, each scaled by what the counter reads for a plain
device copy of known size); null when that summary is absent.

Extras in the same line, one per benchmark configuration: the
Qwen3-235B-A22B-shaped resident stack decode (94 layers x 128 experts, 119 GiB,
94 chained layer calls a step) at B = 1, 8, 32 with Zipf(1.1) routing; int8
group-scaled experts at B = 1, 4, 16, 64; GGUF Q8_0 / Q4_K experts at B = 1, 32;
the Qwen3-30B-A3B-shaped MoE layer prefill (T=512) with its own CPU baseline.
With --per-layer the 384 evaluations also as 48 per-layer calls; --extras adds
the group-64 int8-activation decode, every GGUF type's mat-vec, the wire codec,
residency and the store's layer call with its host work.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
FP32_PEAK_TFLOPS = 157.3
TRAFFIC_SUMMARY = ROOT / "profiles" / "mv_fast_kernel_int4_decode_384experts.md"


def measured_traffic():
    """HBM bytes per launch of the decode mat-vec from the committed counter
    summary (its line `traffic_bytes_per_launch: N`), or None."""
    try:
        m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.]+)", TRAFFIC_SUMMARY.read_text(), re.M)
    except OSError:
        return None
    return float(m.group(1)) if m else None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def expert_bytes(H: int, I: int, gs: int, scale_bytes: int = 2) -> int:
    """Packed nibbles + scales of one expert (gate|up and down)."""
    n = 3 * H * I
    return n // 2 + n // gs * scale_bytes


class Int4Pool:
    """n experts of shape (H, I) resident in HBM: one tensor per part, so that
    expert e's arrays sit at a fixed stride; a device table of moe_q4_expert."""

    def __init__(self, n: int, H: int, I: int, gs: int, seed: int):
        import torch
        from distributedmoellm_amd import _lib
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.n, self.H, self.I, self.gs = n, H, I, gs
        self.gu_w = torch.randint(0, 256, (n, 2 * I, H // 2), dtype=torch.uint8, device="cuda", generator=g)
        self.dn_w = torch.randint(0, 256, (n, H, I // 2), dtype=torch.uint8, device="cuda", generator=g)
        # scales |N(0, 0.02)| / 8 in f16
        self.gu_s = (torch.randn((n, 2 * I, H // gs), device="cuda", generator=g).abs_() * (0.02 / 8)).half()
        self.dn_s = (torch.randn((n, H, I // gs), device="cuda", generator=g).abs_() * (0.02 / 8)).half()
        table = (_lib.Q4Expert * n)()
        for e in range(n):
            table[e] = _lib.Q4Expert(self.gu_w[e].data_ptr(), self.gu_s[e].data_ptr(), self.dn_w[e].data_ptr(),
                                     self.dn_s[e].data_ptr(), 0x88, 1)
        self.table_host = np.frombuffer(bytes(table), np.uint8)
        self.table = torch.from_numpy(self.table_host.copy()).cuda()
        torch.cuda.synchronize()

    @property
    def expert_bytes(self) -> int:
        return expert_bytes(self.H, self.I, self.gs)


class Calls:
    """Pair lists of a sequence of layer calls, uploaded once (device int32/f32)."""

    def __init__(self, calls):
        """calls: list of (eidx[k], rows per expert (list of arrays), weights per expert)."""
        import torch
        from distributedmoellm_amd import kernels
        self.items = []
        parts, spec = [], []
        for eidx, rows, ws in calls:
            poff, prow, pw, rrow, rptr, rpair = kernels.pair_lists(rows, ws)
            spec.append((len(eidx), int(poff[-1]), len(rrow), int(np.diff(poff).max()), int(np.diff(rptr).max())))
            parts += [np.asarray(eidx, np.int32).tobytes(), poff.tobytes(), prow.tobytes(), pw.tobytes(),
                      rrow.tobytes(), rptr.tobytes(), rpair.tobytes()]
        self.buf, addrs = kernels.upload_parts(parts)
        for i, (k, P, nr, mr, mp) in enumerate(spec):
            a = addrs[7 * i:7 * i + 7]
            self.items.append(dict(eidx=a[0], poff=a[1], prow=a[2], pw=a[3], rrow=a[4], rptr=a[5], rpair=a[6],
                                   k=k, P=P, nr=nr, max_rows=mr, max_pairs=mp))


def run_layer(L, pool, x, out, h, y, c, stream, ev=None):
    """gate|up mat-vec, down mat-vec (SiLU on load), combine: one layer call."""
    H, I, gs = pool.H, pool.I, pool.gs
    tab = pool.table.data_ptr()
    if ev is not None:
        ev[0].record()
    rc = L.moe_q4_experts_matvec(x.data_ptr(), H, c["prow"], tab, c["eidx"], c["k"], c["poff"], 0, H, I, gs,
                                 c["max_rows"], h.data_ptr(), 2 * I, stream)
    if ev is not None:
        ev[1].record()
    rc |= L.moe_q4_experts_matvec(h.data_ptr(), 2 * I, None, tab, c["eidx"], c["k"], c["poff"], 1, H, I, gs,
                                  c["max_rows"], y.data_ptr(), H, stream)
    if ev is not None:
        ev[2].record()
    rc |= L.moe_combine(y.data_ptr(), H, c["pw"], c["rrow"], c["rptr"], c["rpair"], c["nr"], c["max_pairs"],
                        out.data_ptr(), H, H, stream)
    if rc:
        from distributedmoellm_amd import _lib
        raise RuntimeError(_lib.last_error())


def decode384(args, L, per_layer=False):
    """One token's 48 x 8 expert evaluations per step, C1 expert shape, from a 1024-expert pool."""
    import torch
    H, I, gs, npool, per_step = 2048, 768, 32, 1024, 384
    log(f"pool: {npool} experts H={H} I={I} gs={gs} ({npool * expert_bytes(H, I, gs) / 1e9:.2f} GB)")
    pool = Int4Pool(npool, H, I, gs, seed=1)
    rng = np.random.default_rng(0)
    nvar = 8
    fused, layered = [], []
    for v in range(nvar):
        eidx = np.sort(rng.choice(npool, per_step, replace=False)).astype(np.int32)
        rows = [np.zeros(1, np.int32) for _ in range(per_step)]
        ws = [rng.random(1).astype(np.float32) for _ in range(per_step)]
        fused.append((eidx, rows, ws))
        for l in range(48):
            sl = slice(8 * l, 8 * l + 8)
            layered.append((eidx[sl], rows[sl], ws[sl]))
    cf, cl = Calls(fused), Calls(layered)
    x = torch.randn((1, H), device="cuda")
    out = torch.zeros((1, H), device="cuda")
    h = torch.empty((per_step, 2 * I), device="cuda")
    y = torch.empty((per_step, H), device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    step_bytes = per_step * pool.expert_bytes + 2 * H * 4
    for i in range(args.warmup):
        run_layer(L, pool, x, out, h, y, cf.items[i % nvar], stream)
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        run_layer(L, pool, x, out, h, y, cf.items[i % nvar], stream, evs[i])
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) / args.steps * 1e3
    gu_ms = np.array([e[0].elapsed_time(e[1]) for e in evs])
    dn_ms = np.array([e[1].elapsed_time(e[2]) for e in evs])
    gu_bytes = per_step * (2 * I * H // 2 + 2 * I * (H // gs) * 2) + H * 4
    dn_bytes = per_step * (H * I // 2 + H * (I // gs) * 2) + per_step * 2 * I * 4
    # the dominant kernel is the gate|up launch's mv_fast_kernel; the down
    # launch runs mv_q4w24_kernel (768-value rows in 24-byte chunks)
    gu_s, dn_s = gu_ms.mean() / 1e3, dn_ms.mean() / 1e3
    res = dict(ms_per_step=ms, value=step_bytes / (ms / 1e3) / 1e9, step_bytes=step_bytes,
               kernel=dict(name="mv_fast_kernel<FmtQ4D, 64, 1, 1, true> (int4 decode mat-vec, integer dot8 on "
                                "activation limbs built once a workgroup; the gate|up launch of moe_q4_experts_matvec: 384 experts x "
                                "[1536 x 2048])",
                           launches=args.steps, avg_us=gu_s * 1e6, bytes_per_launch=gu_bytes,
                           achieved_gbs=gu_bytes / gu_s / 1e9,
                           gate_up_us=float(gu_ms.mean() * 1e3), down_us=float(dn_ms.mean() * 1e3),
                           gate_up_gbs=gu_bytes / gu_s / 1e9, down_gbs=dn_bytes / dn_s / 1e9,
                           down_bytes=dn_bytes))
    res["pool"] = pool
    if not per_layer:
        return res
    # the same evaluations as 48 per-layer calls of 8 experts (decode as it runs layer by layer)
    torch.cuda.synchronize()
    steps = max(2, args.steps // 2)
    for i in range(48):
        run_layer(L, pool, x, out, h, y, cl.items[i], stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        v = s % nvar
        for l in range(48):
            run_layer(L, pool, x, out, h, y, cl.items[v * 48 + l], stream)
    torch.cuda.synchronize()
    ms_l = (time.perf_counter() - t0) / steps * 1e3
    res["per_layer_calls"] = dict(ms_per_token=ms_l, gbs=step_bytes / (ms_l / 1e3) / 1e9, calls_per_token=48)
    return res


def decode384_gs64(args, L):
    """The 384 evaluations per step at groups of 64 through the whole layer
    call (moe_q4_layer_i8: int8 activations, as moelan's _moe_q4i; and
    moe_q4_layer: float activations), each timed per call with HIP events on
    the stream the call launches on."""
    import torch
    H, I, gs, npool, per_step = 2048, 768, 64, 1024, 384
    pool = Int4Pool(npool, H, I, gs, seed=3)
    rng = np.random.default_rng(4)
    nvar = 8
    calls = Calls([(np.sort(rng.choice(npool, per_step, replace=False)).astype(np.int32),
                    [np.zeros(1, np.int32) for _ in range(per_step)],
                    [rng.random(1).astype(np.float32) for _ in range(per_step)]) for _ in range(nvar)])
    x = torch.randn((1, H), device="cuda")
    out = torch.zeros((1, H), device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    step_bytes = per_step * pool.expert_bytes + 2 * H * 4
    res = {}
    for name, fn, need in (("int8_act", L.moe_q4_layer_i8, L.moe_q4_layer_i8_workspace(per_step, H, I, gs)),
                           ("float_act", L.moe_q4_layer, L.moe_q4_layer_workspace(per_step, H, I))):
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")

        def call(c):
            rc = fn(x.data_ptr(), H, pool.table.data_ptr(), c["eidx"], c["k"], c["poff"], c["prow"], c["pw"],
                    c["P"], c["rrow"], c["rptr"], c["rpair"], c["nr"], out.data_ptr(), H, H, I, gs,
                    c["max_rows"], ws.data_ptr(), need, stream)
            if rc:
                from distributedmoellm_amd import _lib
                raise RuntimeError(_lib.last_error())
        for i in range(args.warmup):
            call(calls.items[i % nvar])
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(args.steps):
            call(calls.items[i % nvar])
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        res[name] = dict(ms_per_step=ms, gbs=step_bytes / (ms / 1e3) / 1e9,
                         hbm_frac=step_bytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS)
        log(f"decode384 gs=64 {name}: {ms * 1e3:.1f} us/step, {res[name]['gbs']:.0f} GB/s")
        del ws
    res["bytes_per_step"] = step_bytes
    res["workload"] = ("one token's 384 expert evaluations per layer call, H=2048 I=768, int4 group 64, "
                       "f16 scales, 1024-expert pool; whole call (rounding, gate|up, down, combine)")
    del pool
    torch.cuda.empty_cache()
    return res


GGUF_TYPES = {2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24),
              8: ("Q8_0", 32, 34), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144),
              13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210)}


def gguf_matvec(args, L, target_bytes: int = 256 << 20, cols: int = 2048):
    """Each GGUF block type's decode mat-vec (moe_gguf_matmul_t, one input row)
    on one matrix of rows of 2048 values and about 256 MB: the kernel's
    streaming rate against the HBM roofline. Bytes are the blocks' bytes;
    HIP events around 20 launches on the launch stream."""
    import torch
    stream = torch.cuda.current_stream().cuda_stream
    x = torch.randn((1, cols), device="cuda")
    res = {}
    for qt, (name, per, size) in GGUF_TYPES.items():
        row_bytes = cols // per * size
        O = target_bytes // row_bytes
        raw = torch.randint(0, 256, (O, row_bytes), dtype=torch.uint8, device="cuda")
        y = torch.empty((1, O), device="cuda")
        for _ in range(max(2, args.warmup)):
            rc = L.moe_gguf_matmul_t(x.data_ptr(), 1, raw.data_ptr(), qt, O, cols, y.data_ptr(), stream)
            if rc:
                from distributedmoellm_amd import _lib
                raise RuntimeError(_lib.last_error())
        n = 20
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(n):
            L.moe_gguf_matmul_t(x.data_ptr(), 1, raw.data_ptr(), qt, O, cols, y.data_ptr(), stream)
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) / n * 1e3
        byts = O * row_bytes + cols * 4 + O * 4
        res[name] = dict(us=round(us, 2), bytes=byts, gbs=round(byts / us / 1e3, 1),
                         hbm_frac=round(byts / us / 1e3 / HBM_PEAK_GBS, 4))
        log(f"gguf {name}: {O} x {cols}, {byts / 1e6:.0f} MB in {us:.1f} us = {byts / us / 1e3:.0f} GB/s")
        del raw, y
    torch.cuda.empty_cache()
    res["workload"] = ("one input row against one matrix of rows of 2048 values, about 256 MB of blocks "
                       "(every byte random, so scale fields are arbitrary f16), 20 launches")
    return res


def _time_calls(fn, n, warm=3):
    """Mean milliseconds of fn() over n calls, HIP events on the current stream."""
    import torch
    for _ in range(warm):
        fn(0)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(n):
        fn(i)
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / n


def _check(rc):
    if rc:
        from distributedmoellm_amd import _lib
        raise RuntimeError(_lib.last_error())


def int8_c2(args, L, batches=(1, 4, 16, 64)):
    """Group-scaled int8 experts (H=2048, I=768: gate|up [1536 x 2048], down
    [2048 x 768], group 32, f16 scales |N(0,0.02)|/127, int8 uniform in
    [-127, 127]) applied to B routed rows (moe_q8_matmul_t, the reference's
    q8_matmul_t per matrix): per expert evaluation (two calls, experts cycled
    through a 256-expert, 1.28 GB pool) and the kernel's rate on one stacked
    gate|up matrix of all 256 experts (805 MB, one call). Bytes: int8 values +
    f16 scales (5,013,504 per expert) + activations; flops 2 B 3 H I."""
    import torch
    H, I, gs, n = 2048, 768, 32, 256
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    qgu = torch.randint(-127, 128, (n, 2 * I, H), dtype=torch.int8, device="cuda", generator=g)
    qdn = torch.randint(-127, 128, (n, H, I), dtype=torch.int8, device="cuda", generator=g)
    sgu = (torch.randn((n, 2 * I, H // gs), device="cuda", generator=g).abs_() * (0.02 / 127)).half()
    sdn = (torch.randn((n, H, I // gs), device="cuda", generator=g).abs_() * (0.02 / 127)).half()
    stream = torch.cuda.current_stream().cuda_stream
    ebytes = 3 * H * I + 3 * H * I // gs * 2
    res = {}
    for B in batches:
        x = torch.randn((B, H), device="cuda")
        a = torch.randn((B, I), device="cuda")
        ygu = torch.empty((B, 2 * I), device="cuda")
        ydn = torch.empty((B, H), device="cuda")

        def expert(i):
            e = (i * 37) % n
            _check(L.moe_q8_matmul_t(x.data_ptr(), B, qgu[e].data_ptr(), sgu[e].data_ptr(), 1, 2 * I, H, gs,
                                     ygu.data_ptr(), stream))
            _check(L.moe_q8_matmul_t(a.data_ptr(), B, qdn[e].data_ptr(), sdn[e].data_ptr(), 1, H, I, gs,
                                     ydn.data_ptr(), stream))
        ms = _time_calls(expert, 128)
        byts = ebytes + B * (H + I) * 4 * 2
        flops = 2.0 * B * 3 * H * I
        ybig = torch.empty((B, n * 2 * I), device="cuda")

        def stacked(i):
            _check(L.moe_q8_matmul_t(x.data_ptr(), B, qgu.data_ptr(), sgu.data_ptr(), 1, n * 2 * I, H, gs,
                                     ybig.data_ptr(), stream))
        ms_big = _time_calls(stacked, 10)
        big_bytes = n * 2 * I * (H + H // gs * 2) + B * (H + n * 2 * I) * 4
        big_flops = 2.0 * B * n * 2 * I * H
        res[f"B{B}"] = dict(us_per_expert=round(ms * 1e3, 2), gbs_per_expert=round(byts / ms / 1e6, 1),
                            hbm_frac_per_expert=round(byts / ms / 1e6 / HBM_PEAK_GBS, 4),
                            fp32_frac_per_expert=round(flops / ms / 1e9 / FP32_PEAK_TFLOPS, 4),
                            stacked_us=round(ms_big * 1e3, 1), stacked_gbs=round(big_bytes / ms_big / 1e6, 1),
                            stacked_hbm_frac=round(big_bytes / ms_big / 1e6 / HBM_PEAK_GBS, 4),
                            stacked_fp32_frac=round(big_flops / ms_big / 1e9 / FP32_PEAK_TFLOPS, 4),
                            bound="hbm" if B <= 4 else "fp32")
        log(f"int8 B={B}: {ms * 1e3:.1f} us/expert ({byts / ms / 1e6:.0f} GB/s), stacked gate|up "
            f"{big_bytes / ms_big / 1e6:.0f} GB/s ({big_flops / ms_big / 1e9:.1f} TFLOP/s)")
        del x, a, ygu, ydn, ybig
    res["workload"] = ("C2: int8 group-32 experts H=2048 I=768, f16 scales, B routed rows; per expert = the two "
                       "q8_matmul_t calls of an expert evaluation from a 256-expert (1.28 GB) pool; stacked = one "
                       "call over all 256 experts' gate|up rows (805 MB)")
    del qgu, qdn, sgu, sdn
    torch.cuda.empty_cache()
    return res


def gguf_c3(args, L, batches=(1, 32)):
    """GGUF experts at the Qwen3-30B-A3B shape: gate and up [768 x 2048] and
    down [2048 x 768] in Q8_0 (34-byte blocks of 32) and Q4_K (144-byte
    superblocks of 256), B routed rows (moe_gguf_matmul_t, the reference's
    gguf_matmul_t per matrix): per expert evaluation (three calls) cycled
    through a pool beyond the 256 MB MALL. Blocks are random bytes with their
    f16 d (and dmin) fields set to |N(0, 0.01)|. Bytes: the blocks +
    activations."""
    import torch
    H, I = 2048, 768
    stream = torch.cuda.current_stream().cuda_stream
    res = {}
    for qt, name, n in ((8, "Q8_0", 128), (12, "Q4_K", 256)):
        _, per, size = GGUF_TYPES[qt]
        g = torch.Generator(device="cuda")
        g.manual_seed(31 + qt)

        def blocks(O, cols):
            raw = torch.randint(0, 256, (n, O, cols // per, size), dtype=torch.uint8, device="cuda", generator=g)
            d = (torch.randn((n, O, cols // per), device="cuda", generator=g).abs_() * 0.01).half()
            raw[..., 0:2] = d.view(torch.uint8).view(n, O, cols // per, 2)
            if qt == 12:   # dmin
                dm = (torch.randn((n, O, cols // per), device="cuda", generator=g).abs_() * 0.01).half()
                raw[..., 2:4] = dm.view(torch.uint8).view(n, O, cols // per, 2)
            return raw.view(n, O, cols // per * size)
        gate, up, down = blocks(I, H), blocks(I, H), blocks(H, I)
        ebytes = (2 * I * (H // per) + H * (I // per)) * size
        for B in batches:
            x = torch.randn((B, H), device="cuda")
            a = torch.randn((B, I), device="cuda")
            yg = torch.empty((B, I), device="cuda")
            yu = torch.empty((B, I), device="cuda")
            yd = torch.empty((B, H), device="cuda")

            def expert(i):
                e = (i * 37) % n
                _check(L.moe_gguf_matmul_t(x.data_ptr(), B, gate[e].data_ptr(), qt, I, H, yg.data_ptr(), stream))
                _check(L.moe_gguf_matmul_t(x.data_ptr(), B, up[e].data_ptr(), qt, I, H, yu.data_ptr(), stream))
                _check(L.moe_gguf_matmul_t(a.data_ptr(), B, down[e].data_ptr(), qt, H, I, yd.data_ptr(), stream))
            ms = _time_calls(expert, 128)
            byts = ebytes + B * (2 * H + 3 * I) * 4 + B * (2 * I + H) * 4
            flops = 2.0 * B * 3 * H * I
            res[f"{name}_B{B}"] = dict(us_per_expert=round(ms * 1e3, 2), gbs=round(byts / ms / 1e6, 1),
                                       hbm_frac=round(byts / ms / 1e6 / HBM_PEAK_GBS, 4),
                                       fp32_frac=round(flops / ms / 1e9 / FP32_PEAK_TFLOPS, 4),
                                       bytes_per_expert=ebytes)
            log(f"gguf {name} B={B}: {ms * 1e3:.1f} us/expert, {byts / ms / 1e6:.0f} GB/s")
            del x, a, yg, yu, yd
        del gate, up, down
    res["workload"] = ("C3: GGUF Q8_0 / Q4_K experts, gate and up [768 x 2048], down [2048 x 768], three "
                       "gguf_matmul_t calls per expert evaluation, B routed rows, pools of 128 (Q8_0, 642 MB) and "
                       "256 (Q4_K, 680 MB) experts")
    torch.cuda.empty_cache()
    return res


def wire_codec(args, L, n: int = 8192, d: int = 4096):
    """Wire encode (moe_wire_encode) of an [n, d] f32 block in HBM (128 MB) to
    int8 + scales and to f16, and the int8 decode back: bytes read + written
    over HIP-event time of 20 launches each."""
    import torch
    stream = torch.cuda.current_stream().cuda_stream
    a = torch.randn((n, d), device="cuda")
    q = torch.empty((n, d), dtype=torch.int8, device="cuda")
    h = torch.empty((n, d), dtype=torch.float16, device="cuda")
    sc = torch.empty((n, d // 64), device="cuda")
    back = torch.empty((n, d), device="cuda")
    calls = {
        "encode_int8": (lambda: L.moe_wire_encode(a.data_ptr(), d, None, n, d, 2, q.data_ptr(), sc.data_ptr(), stream),
                        n * d * 4 + n * d + n * d // 64 * 4),
        "encode_f16": (lambda: L.moe_wire_encode(a.data_ptr(), d, None, n, d, 1, h.data_ptr(), None, stream),
                       n * d * 4 + n * d * 2),
        "decode_int8": (lambda: L.moe_wire_decode(q.data_ptr(), sc.data_ptr(), 2, n, d, None, back.data_ptr(), d,
                                                  stream), n * d + n * d // 64 * 4 + n * d * 4),
    }
    res = {}
    for name, (fn, byts) in calls.items():
        for _ in range(3):
            if fn():
                from distributedmoellm_amd import _lib
                raise RuntimeError(_lib.last_error())
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(20):
            fn()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) / 20 * 1e3
        res[name] = dict(us=round(us, 2), bytes=byts, gbs=round(byts / us / 1e3, 1),
                         hbm_frac=round(byts / us / 1e3 / HBM_PEAK_GBS, 4))
        log(f"wire {name}: {us:.1f} us, {byts / us / 1e3:.0f} GB/s")
    res["workload"] = f"[{n}, {d}] f32 activations in HBM (128 MB), 20 launches each"
    del a, q, h, sc, back
    torch.cuda.empty_cache()
    return res


def residency(args, L, n: int = 64):
    """Experts from a colibri int4 container into HBM: n experts of the
    Qwen3-30B-A3B shape (H=2048, I=768, group 32, f32 scales as colibri stores
    them) written to a temporary directory (so in the page cache), then
    ExpertStore.pin of all of them timed: memory-mapped views, one
    host-to-device copy per array. Bound by the host link, not HBM."""
    import json as _json
    import tempfile
    import torch
    from safetensors.numpy import save_file
    from distributedmoellm_amd import experts as X
    from distributedmoellm_amd import sources as S
    H, I, gs = 2048, 768, 32
    rng = np.random.default_rng(9)
    with tempfile.TemporaryDirectory() as d:
        tensors = {}
        for e in range(n):
            p = f"model.layers.0.mlp.experts.{e}"
            tensors[f"{p}.merged_weight"] = rng.integers(0, 256, 3 * H * I // 2, dtype=np.uint8)
            tensors[f"{p}.qs"] = rng.random(3 * H * I // gs, dtype=np.float32)
        save_file(tensors, f"{d}/model.safetensors")
        del tensors
        with open(f"{d}/config.json", "w") as f:
            _json.dump({"model_type": "qwen3_moe", "hidden_size": H, "moe_intermediate_size": I, "num_experts": n,
                        "num_hidden_layers": 1}, f)
        with open(f"{d}/qwen36_meta.json", "w") as f:
            _json.dump({"ebits": 4, "expert_gs": gs}, f)
        src = S.CheckpointSource(d)
        X.ExpertStore([src]).pin([(0, 0)])           # the staging buffers and the copy path
        torch.cuda.synchronize()
        keys = [(0, e) for e in range(n)]
        times = []
        for _ in range(2):   # first into new device memory, then again after forget (memory torch keeps)
            store = X.ExpertStore([src])
            t0 = time.perf_counter()
            store.pin(keys)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
            byts = store.resident_bytes()
            store.forget(keys)
            del store
        del src
    torch.cuda.empty_cache()
    res = dict(experts=n, bytes=byts, seconds=round(times[0], 4), gbs=round(byts / times[0] / 1e9, 2),
               seconds_warm=round(times[1], 4), gbs_warm=round(byts / times[1] / 1e9, 2), bound="host link",
               workload=f"{n} colibri int4 experts (H=2048 I=768 gs=32, f32 scales, {byts / 1e6:.0f} MB) "
                        "pinned from a page-cached container; gbs into new device memory, gbs_warm into "
                        "memory the allocator already holds")
    log(f"residency: {n} experts, {byts / 1e6:.0f} MB in {times[0] * 1e3:.1f} ms = {res['gbs']} GB/s "
        f"(again: {times[1] * 1e3:.1f} ms = {res['gbs_warm']} GB/s)")
    return res


def store_call(args, L, E: int = 128, H: int = 2048, I: int = 768, gs: int = 32, k: int = 8,
               batches=(1, 8, 512), n: int = 50):
    """ExpertStore.compute as moelan's callers use it (moelan/experts.py:641-753,
    model.py:468): one layer's routed experts (Qwen3-30B-A3B shape, 128 int4
    experts resident, top-8 Zipf(1.1) routing) for B tokens, host work
    included -- the pair lists built and uploaded, the expert table, the
    workspace. ``wall_us``: each call enqueued and waited for, one at a time;
    ``gpu_us``: HIP events around the same calls back to back (the device
    time, host gaps included); ``kernel_us``: the same layer call on pair lists
    already on the device (B <= 8) or the prompt layer call (B = 512, router
    included), the device work alone."""
    import torch
    from distributedmoellm_amd import experts as X
    from distributedmoellm_amd import kernels as K
    rng = np.random.default_rng(17)
    store = X.ExpertStore({(0, e): X.synthetic_expert(H, I, "int4", gs, rng) for e in range(E)})
    res = {}
    for B in batches:
        eidx, rows, ws = zipf_calls(rng, B, E, k)
        groups = list(zip(eidx.tolist(), rows, ws))
        x = torch.randn(B, H, device="cuda")
        for _ in range(3):
            store.compute(0, x, groups)
        torch.cuda.synchronize()
        wall = []
        for _ in range(n):
            t0 = time.perf_counter()
            store.compute(0, x, groups)
            torch.cuda.synchronize()
            wall.append(time.perf_counter() - t0)
        gpu = _time_calls(lambda i: store.compute(0, x, groups), n)
        if B <= 8:
            items = [(K.q4_expert_ptrs(store.get((0, int(e)))), r, w) for e, r, w in groups]
            meta = K.LayerMeta([p for p, _, _ in items], rows, ws)
            out = torch.zeros(B, H, device="cuda")
            ws_t = torch.empty(L.moe_q4_layer_workspace(max(meta.P, 1), H, I), dtype=torch.uint8, device="cuda")
            kern = _time_calls(lambda i: K.moe_q4_run(x, meta, H, I, gs, out, workspace=ws_t), n)
        else:
            table = store.layer_table(0, E)
            router = torch.randn(E, H, device="cuda") * 0.05
            out = torch.empty(B, H, device="cuda")
            ws_t = torch.empty(L.moe_prefill_workspace(B, E, k, H, I), dtype=torch.uint8, device="cuda")
            kern = _time_calls(lambda i: K.prefill_layer(x, router, table, k, True, H, I, gs, out=out,
                                                         workspace=ws_t), n)
        wall.sort()
        res[f"B{B}"] = dict(experts=len(groups), wall_us=round(wall[len(wall) // 2] * 1e6, 1),
                            gpu_us=round(gpu * 1e3, 1), kernel_us=round(kern * 1e3, 1))
        log(f"store B={B}: {len(groups)} experts, {res[f'B{B}']['wall_us']} us a call waited for, "
            f"{res[f'B{B}']['gpu_us']} us back to back, device work alone {res[f'B{B}']['kernel_us']} us")
    res["workload"] = (f"ExpertStore.compute over {E} resident int4 experts (H={H} I={I} gs={gs}, f16 scales), "
                       f"top-{k} Zipf(1.1) routing of B tokens; median wall time of {n} calls each waited for")
    del store
    torch.cuda.empty_cache()
    return res


def cpu_baseline_decode(seconds: float = 12.0):
    """The reference's fused layer kernel restated in C/OpenMP (oracle/cpuref.c)
    on the host cores: one token's 384 experts per call from a pool of 64
    experts (170 MB, beyond the last-level cache), f32 scales as the reference
    requires; GB/s counted with the same algorithmic bytes as the GPU."""
    from oracle import build_cpuref
    L = build_cpuref.load()
    H, I, gs, npool, per_call = 2048, 768, 32, 64, 384
    rng = np.random.default_rng(2)
    gu = [rng.integers(0, 256, (2 * I, H // 2), dtype=np.uint8) for _ in range(npool)]
    gs_ = [(np.abs(rng.normal(0, 0.02, (2 * I, H // gs))) / 8).astype(np.float16).astype(np.float32)
           for _ in range(npool)]
    dn = [rng.integers(0, 256, (H, I // 2), dtype=np.uint8) for _ in range(npool)]
    ds_ = [(np.abs(rng.normal(0, 0.02, (H, I // gs))) / 8).astype(np.float16).astype(np.float32)
           for _ in range(npool)]
    addr = lambda a: a.__array_interface__["data"][0]
    ptrs = np.array([[addr(gu[e]), addr(gs_[e]), addr(dn[e]), addr(ds_[e])] for e in range(npool)], np.uint64)
    x = rng.standard_normal((1, H)).astype(np.float32)
    poff = np.arange(per_call + 1, dtype=np.int64)
    prow = np.zeros(per_call, np.int64)
    pw = rng.random(per_call).astype(np.float32)
    xors = np.full(per_call, 0x88, np.uint8)
    out = np.zeros((1, H), np.float32)

    def call(i):
        sel = (np.arange(per_call) + i * 7) % npool
        pt = np.ascontiguousarray(ptrs[sel].reshape(-1))
        L.ref_moe_q4(x.ctypes.data, 1, pt.ctypes.data, xors.ctypes.data, poff.ctypes.data, prow.ctypes.data,
                     pw.ctypes.data, per_call, per_call, H, I, gs, out.ctypes.data)
    call(0)
    rounds, total_calls = [], 0
    for _ in range(3):   # median of 3 rounds, as the reference's bench_expert (moelan/experts.py:366-373)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds / 3:
            call(total_calls + n + 1)
            n += 1
        dt = time.perf_counter() - t0
        total_calls += n
        rounds.append(n * per_call * expert_bytes(H, I, gs) / dt / 1e9)
    value = float(np.median(rounds))
    return dict(value=value, unit="GB/s", cores=int(L.ref_threads()), kind="port",
                rounds_gbs=[round(r, 2) for r in rounds], host=host_info(),
                sample=f"median of 3 rounds of ~{seconds / 3:.0f} s ({total_calls} calls in all) of one token's 384 "
                       f"experts (H=2048 I=768 gs=32) from a 64-expert host pool (170 MB); oracle/cpuref.c "
                       f"ref_moe_q4 (the _moe_q4 loop structure), OpenMP over {int(L.ref_threads())} threads")


def host_info() -> dict:
    """The host the CPU baseline ran on: CPU model, the cores this process may
    run on, and the thread settings OpenMP / BLAS read."""
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(cpu_model=model, affinity_cores=len(os.sched_getaffinity(0)),
                OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS"),
                OPENBLAS_NUM_THREADS=os.environ.get("OPENBLAS_NUM_THREADS"))


def zipf_calls(rng, B: int, E: int = 128, k: int = 8, s: float = 1.1):
    """Top-k per token without replacement from p_r ~ r^-s over a seeded permutation
    of expert ids; weights softmax(N(0,1)). Returns (eidx, rows per expert, weights)."""
    perm = rng.permutation(E)
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    picks = {}
    for t in range(B):
        ex = perm[rng.choice(E, size=k, replace=False, p=p)]
        w = np.exp(rng.standard_normal(k))
        w /= w.sum()
        for e, wt in zip(ex, w):
            picks.setdefault(int(e), []).append((t, float(wt)))
    eidx = np.array(sorted(picks), np.int32)
    rows = [np.array([t for t, _ in picks[e]], np.int32) for e in eidx]
    ws = [np.array([w for _, w in picks[e]], np.float32) for e in eidx]
    return eidx, rows, ws


def stack_decode(args, L, batches=(1, 8, 32)):
    """Qwen3-235B-A22B-shaped expert stack resident in HBM (94 layers x 128
    experts, H=4096, I=1536, int4 group 32, f16 scales, 119 GiB), one
    continuous-batching decode step per timed iteration at B tokens: 94
    layer calls in sequence (moe_q4_layer), each on the previous layer's output
    (the residual stream x += MoE(x), in place), top-8 routing from a seeded
    Zipf(1.1) expert popularity per layer. Bytes per step: the packed weights
    and scales of every distinct (layer, expert) touched, plus activations."""
    import torch
    H, I, gs, E, layers = 4096, 1536, 32, 128, 94
    log(f"stack: {layers} layers x {E} experts H={H} I={I} ({layers * E * expert_bytes(H, I, gs) / 2**30:.1f} GiB)")
    pools = [Int4Pool(E, H, I, gs, seed=100 + l) for l in range(layers)]
    stream = torch.cuda.current_stream().cuda_stream
    res = {}
    for B in batches:
        rng = np.random.default_rng(B)
        nvar = 2
        calls = Calls([zipf_calls(rng, B) for _ in range(nvar * layers)])
        dist = np.array([calls.items[i]["k"] for i in range(nvar * layers)]).reshape(nvar, layers)
        rows_max = max(c["max_rows"] for c in calls.items)
        step_bytes = dist.sum(1) * expert_bytes(H, I, gs) + 2 * layers * B * H * 4
        Pmax = max(c["P"] for c in calls.items)
        need = L.moe_q4_layer_workspace(Pmax, H, I)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        x = torch.randn((B, H), device="cuda")

        def step(v, stream=stream):
            for l in range(layers):
                c = calls.items[v * layers + l]
                rc = L.moe_q4_layer(x.data_ptr(), H, pools[l].table.data_ptr(), c["eidx"], c["k"], c["poff"],
                                    c["prow"], c["pw"], c["P"], c["rrow"], c["rptr"], c["rpair"], c["nr"],
                                    x.data_ptr(), H, H, I, gs, c["max_rows"], ws.data_ptr(), need, stream)
                if rc:
                    from distributedmoellm_amd import _lib
                    raise RuntimeError(_lib.last_error())
        for v in range(nvar):
            x.normal_()
            step(v)
        torch.cuda.synchronize()
        nsteps = max(4, min(args.steps, 20))
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nsteps)]
        for s_ in range(nsteps):
            x.normal_()          # a fresh token batch: outside the timed events
            evs[s_][0].record()
            step(s_ % nvar)
            evs[s_][1].record()
        torch.cuda.synchronize()
        ms = float(np.median([a.elapsed_time(b) for a, b in evs]))
        # the same steps captured as HIP graphs (one per routing variant) and replayed
        graphs = []
        for v in range(nvar if not args.no_graph else 0):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(v, torch.cuda.current_stream().cuda_stream)
            graphs.append(g)
        torch.cuda.synchronize()
        gevs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nsteps)]
        for s_ in range(nsteps if graphs else 0):
            x.normal_()
            gevs[s_][0].record()
            graphs[s_ % nvar].replay()
            gevs[s_][1].record()
        torch.cuda.synchronize()
        ms_graph = float(np.median([a.elapsed_time(b) for a, b in gevs])) if graphs else float("nan")
        del graphs
        avg_bytes = float(step_bytes.mean())
        key = f"B{B}"
        res[key] = dict(ms_per_step=ms, ms_per_step_graph=ms_graph, gbs=avg_bytes / (ms / 1e3) / 1e9,
                        gbs_graph=avg_bytes / (ms_graph / 1e3) / 1e9, bytes_per_step=avg_bytes,
                        hbm_frac=avg_bytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS,
                        experts_per_layer=float(dist.mean()), max_rows_per_expert=int(rows_max),
                        peak_ms=avg_bytes / (HBM_PEAK_GBS * 1e9) * 1e3,
                        target_ms_70pct=avg_bytes / (0.7 * HBM_PEAK_GBS * 1e9) * 1e3,
                        launches_per_layer=3 if rows_max == 1 else 5)
        log(f"stack B={B}: {ms:.3f} ms/step ({ms_graph:.3f} as a graph), {res[key]['gbs']:.0f} GB/s "
            f"({res[key]['hbm_frac'] * 100:.1f}% of HBM), "
            f"{dist.mean():.1f} experts/layer, hottest {rows_max} rows")
        del ws
    res["workload"] = ("Qwen3-235B-A22B-shaped stack: 94 sequential layer calls per step (x += MoE(x)), 128 experts "
                       "a layer, H=4096 I=1536 int4 g32 f16 scales (119 GiB resident), top-8 Zipf(1.1) routing; "
                       "median of timed steps, HIP events")
    del pools
    torch.cuda.empty_cache()
    return res


def prefill_c4(args, L):
    """Qwen3-30B-A3B-shaped MoE layer prefill: T=512 tokens, 128 experts (H=2048,
    I=768, int4 g32, f16 scales), f32 router, softmax top-8 renormalised. Four
    layers' experts (1.36 GB) are cycled so each step streams its 340 MB of
    expert weights from HBM rather than the 256 MB MALL."""
    import torch
    T, H, I, gs, E, k, nlayers = 512, 2048, 768, 32, 128, 8, 4
    pools = [Int4Pool(E, H, I, gs, seed=200 + l) for l in range(nlayers)]
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    routers = [torch.randn((E, H), device="cuda", generator=g) * 0.02 for _ in range(nlayers)]
    x = torch.randn((T, H), device="cuda", generator=g)
    out = torch.empty((T, H), device="cuda")
    need = L.moe_prefill_workspace(T, E, k, H, I)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def step(i):
        l = i % nlayers
        rc = L.moe_prefill_layer(x.data_ptr(), H, routers[l].data_ptr(), T, E, k, 1, pools[l].table.data_ptr(), H, I,
                                 gs, out.data_ptr(), H, ws.data_ptr(), ws.numel(), stream)
        if rc:
            from distributedmoellm_amd import _lib
            raise RuntimeError(_lib.last_error())
    for i in range(max(args.warmup, nlayers)):
        step(i)
    torch.cuda.synchronize()
    steps = max(8, args.steps)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        evs[i][0].record()
        step(i)
        evs[i][1].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) / steps * 1e3
    ev_ms = float(np.mean([a.elapsed_time(b) for a, b in evs]))
    flops = T * k * 2 * 3 * H * I + 2 * T * H * E
    wbytes = E * expert_bytes(H, I, gs)
    res = dict(ms_per_layer=ev_ms, wall_ms_per_layer=wall_ms, tokens_per_s=T / (ev_ms / 1e3),
               tflops=flops / (ev_ms / 1e3) / 1e12, mfma_frac=flops / (ev_ms / 1e3) / 1e12 / BF16_PEAK_TFLOPS,
               hbm_gbs=(wbytes + 2 * T * H * 4) / (ev_ms / 1e3) / 1e9,
               hbm_frac=(wbytes + 2 * T * H * 4) / (ev_ms / 1e3) / 1e9 / HBM_PEAK_GBS,
               hbm_floor_us=wbytes / (HBM_PEAK_GBS * 1e9) * 1e6, mfma_floor_us=flops / (BF16_PEAK_TFLOPS * 1e12) * 1e6,
               config="T=512, 128 experts H=2048 I=768 int4 g32 f16 scales, top-8 softmax renormalised, "
                      "f16 MFMA operands with f32 accumulation")
    res["attainable_frac"] = max(res["hbm_floor_us"], res["mfma_floor_us"]) / (ev_ms * 1e3)
    del pools
    torch.cuda.empty_cache()
    return res


def cpu_baseline_prefill(seconds: float = 6.0):
    """The reference's prompt path restated on the host: per expert, widen the
    int4 matrix to f32 and multiply with BLAS (numpy), as moelan/experts.py:216-219
    with moelan/kernels.py:971-973; a bounded sample of experts."""
    from oracle import restate as R
    H, I, gs, rows = 2048, 768, 32, 32
    rng = np.random.default_rng(3)
    n, t0 = 0, time.perf_counter()
    x = rng.standard_normal((rows, H)).astype(np.float32)
    mats = [(rng.integers(0, 256, (2 * I, H // 2), dtype=np.uint8),
             (np.abs(rng.normal(0, 0.02, (2 * I, H // gs))) / 8).astype(np.float32),
             rng.integers(0, 256, (H, I // 2), dtype=np.uint8),
             (np.abs(rng.normal(0, 0.02, (H, I // gs))) / 8).astype(np.float32)) for _ in range(4)]
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        gr, gsc, dr, dsc = mats[n % 4]
        h = x @ R.q4_dequant(gr, gsc, gs, False).T
        a = h[:, :I] / (1 + np.exp(-h[:, :I])) * h[:, I:]
        _ = a @ R.q4_dequant(dr, dsc, gs, False).T
        n += 1
    dt = time.perf_counter() - t0
    per_expert = dt / n
    # a layer of 512 tokens x top-8 = 4096 rows over 128 experts, 32 rows each
    layer_s = per_expert * 128
    return dict(tokens_per_s=512 / layer_s, layer_ms=layer_s * 1e3, experts_timed=n,
                threads=os.environ.get("OMP_NUM_THREADS") or str(len(os.sched_getaffinity(0))),
                host=host_info(),
                kind="port", sample=f"{n} experts x 32 rows: numpy widen (oracle q4_dequant) + BLAS x @ W.T, "
                                    f"scaled to a 128-expert layer")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--extras", action="store_true",
                    help="also run the group-64 int8/float decode, GGUF, wire, residency and store-call measurements "
                         "(each has its own --only part; kept out of the default run to keep it short)")
    ap.add_argument("--per-layer", action="store_true", help="also time the 384 evaluations as 48 per-layer calls")
    ap.add_argument("--batches", default="1,8,32", help="token batches of the 235B-shaped stack decode")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-graph", action="store_true", help="skip the graph-replay figure of the stack decode "
                                                            "(for counter runs)")
    ap.add_argument("--only", default="", help="comma list of parts to run alone: decode, stack, int8, gguf_c3, prefill, decode_i8, gguf, wire, "
                                                "residency, store, copy "
                                                "(for counter and trace runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path's kernels run on one MI355X and --gpus {args.gpus} "
              f"is not supported: the routed-expert path would shard by expert, one share per GPU, "
              f"which this build does not run.", file=sys.stderr)
        return 2
    import torch
    from distributedmoellm_amd import _lib, kernels
    if not kernels.ENABLED:
        raise SystemExit(f"HIP kernels unavailable: {kernels.WHY_DISABLED}")
    L = _lib.lib()
    info = _lib.device_info(torch.cuda.current_device())
    log(f"device {info}")

    only = set(filter(None, args.only.split(",")))
    if only:
        res = {}
        if "decode" in only:
            r = decode384(args, L)
            r.pop("pool")
            res["decode"] = r
        if "prefill" in only:
            res["prefill"] = prefill_c4(args, L)
        if "decode_i8" in only:
            res["decode_i8"] = decode384_gs64(args, L)
        if "gguf" in only:
            res["gguf"] = gguf_matvec(args, L)
        if "wire" in only:
            res["wire"] = wire_codec(args, L)
        if "residency" in only:
            res["residency"] = residency(args, L)
        if "store" in only:
            res["store"] = store_call(args, L)
        if "int8" in only:
            res["int8_c2"] = int8_c2(args, L)
        if "gguf_c3" in only:
            res["gguf_c3"] = gguf_c3(args, L)
        if "stack" in only:
            res["stack"] = stack_decode(args, L, tuple(int(b) for b in args.batches.split(",")))
        if "copy" in only:   # a plain device copy of known size (calibrates the traffic counters)
            import torch
            a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
            b = torch.empty_like(a)
            torch.cuda.synchronize()
            for _ in range(3):
                b.copy_(a)
            torch.cuda.synchronize()
            res["copy_bytes"] = a.numel()
        print(json.dumps(res, default=float))
        return 0

    r = decode384(args, L, per_layer=args.per_layer)
    log(f"decode384: {r['ms_per_step']:.3f} ms/step, {r['value']:.0f} GB/s; kernel {r['kernel']['achieved_gbs']:.0f} GB/s")
    del r["pool"]
    torch.cuda.empty_cache()
    extras = {}
    if "per_layer_calls" in r:
        extras["per_layer_calls"] = r.pop("per_layer_calls")
    if args.extras:
        extras["decode384_gs64"] = decode384_gs64(args, L)
        extras["gguf_matvec"] = gguf_matvec(args, L)
        extras["wire"] = wire_codec(args, L)
        extras["residency"] = residency(args, L)
        extras["store"] = store_call(args, L)
    log("C5: Qwen3-235B-A22B-shaped stack decode ...")
    extras["stack_235b"] = stack_decode(args, L, tuple(int(b) for b in args.batches.split(",")))
    log("C2: int8 experts ...")
    extras["int8_c2"] = int8_c2(args, L)
    log("C3: GGUF experts ...")
    extras["gguf_c3"] = gguf_c3(args, L)
    log("prefill (Qwen3-30B-A3B layer, T=512) ...")
    pf = prefill_c4(args, L)
    log(f"prefill: {pf['ms_per_layer'] * 1e3:.1f} us/layer, {pf['tokens_per_s'] / 1e6:.2f} M tok/s, "
        f"MFMA {pf['mfma_frac'] * 100:.1f}%, HBM {pf['hbm_frac'] * 100:.1f}%")
    extras["prefill_c4"] = pf
    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline_decode()
        log(f"cpu baseline: {cpu['value']:.1f} GB/s on {cpu['cores']} threads")
        pf["cpu_baseline"] = cpu_baseline_prefill()
        log(f"cpu prefill baseline: {pf['cpu_baseline']['tokens_per_s']:.0f} tok/s")
    k = r["kernel"]
    traffic = measured_traffic()
    line = {
        "metric": "int4 expert mat-vec HBM GB/s (% peak); MoE-layer prefill tokens/sec on 1 GPU",
        "value": round(r["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x f32 activations (both mat-vec launches: i4 dot8 of the nibbles with exact "
                 "23-bit fixed-point activation limbs per 32/16-value run, i32 sums, f32 group scales and "
                 "accumulation)",
        "data": "synthetic (seeded uniform nibbles, |N(0,0.02)|/8 f16 scales, N(0,1) activations)",
        "config": {"workload": "int4 expert decode mat-vec: one token's 384 routed-expert evaluations "
                               "(48 layers x top-8) per fused call, Qwen3-30B-A3B expert shape H=2048 I=768, "
                               "int4 group 32, f16 scales, from a 1024-expert HBM pool (2.7 GB)",
                   "experts_per_step": 384, "rows_per_expert": 1, "bytes_per_step": r["step_bytes"]},
        "hbm_frac": round(r["value"] / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(k["achieved_gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(k["achieved_gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": k["name"], "avg_launch_us": round(k["avg_us"], 2),
                     "bytes_per_launch": k["bytes_per_launch"],
                     "gate_up": {"us": round(k["gate_up_us"], 2), "gbs": round(k["gate_up_gbs"], 1)},
                     "down": {"kernel": "mv_q4w24_kernel<16, 2, 3> (the down launch: 384 experts x [2048 x 768], rows through an LDS ring)",
                              "us": round(k["down_us"], 2), "gbs": round(k["down_gbs"], 1),
                              "bytes_per_launch": k["down_bytes"],
                              "frac": round(k["down_gbs"] / HBM_PEAK_GBS, 4)}},
        "cpu_baseline": cpu,
        "extras": extras,
        "device": info,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Benchmark of the MI355X fused-turboquant KV-cache hot path (one GPU).

One step = the BASELINE workload on one GPU, inputs resident in HBM:
  * config 2: fused 3-bit encode of K and of V, each [32768, 8, 128] bf16
    (262 144 vectors per tensor), TurboQuantMSE(128, bits=3, seed=42);
  * config 3: one paged decode-attention step over the 3-bit compressed
    cache (B=32, Hq=32, Hkv=8, d=128, ctx 8192, page 16), when the paged
    kernel is built.
``value`` is the encode throughput in GB/s of bf16 input consumed.  Kernel
times come from HIP events on the stream the kernels are launched on (torch's
current stream, which the library launches on).

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "fused-turboquant_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD published


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def time_launches(fn, iters, torch):
    """Average device time of one fn() call, from HIP events on the current stream."""
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(iters):
        fn()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / iters  # us


def cpu_baseline_encode(n_vec=65536, d=128, bits=3):
    """Oracle (numpy restatement of the reference's unfused path) encode on the host."""
    import numpy as np
    import torch
    from oracle import tq_oracle as O
    from fused_turboquant.core.hadamard import generate_rht_signs
    from fused_turboquant.core.lloyd_max import compute_lloyd_max_codebook
    g = torch.Generator().manual_seed(0)
    x = torch.randn(n_vec, d, generator=g).to(torch.bfloat16).float().numpy()
    s = generate_rht_signs(d, 42).numpy()
    bnd = compute_lloyd_max_codebook(d, bits)[0].astype(np.float32)
    O.encode(x[:1024], s, bnd, bits)
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        O.encode(x, s, bnd, bits)
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    return n_vec * d * 2 / t / 1e9, f"{n_vec} vectors x d={d} bf16, 3-bit encode, median of 5"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 256 MiB device-to-device copy (calibrates rocprof byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this path runs on one GPU; --gpus above 1 is not supported "
                          "(the hot path has no collectives; each GPU would run the same kernels on its own shard)"}))
        sys.exit(2)

    import torch
    from fused_turboquant import TurboQuantMSE

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    d, bits, T, H = 128, 3, 32768, 8
    n = T * H
    log(f"[bench] config2 encode: [{T},{H},{d}] bf16 3-bit, K and V")
    g = torch.Generator(device="cpu").manual_seed(0)
    sc = torch.exp(0.5 * torch.randn(d, generator=torch.Generator().manual_seed(1)))
    k = (torch.randn(T, H, d, generator=g) * sc).to(torch.bfloat16).to(dev)
    v = (torch.randn(T, H, d, generator=g) * sc).to(torch.bfloat16).to(dev)
    tq = TurboQuantMSE(d, bits=bits, seed=42, device=dev)
    ck = tq.encode(k)
    cv = tq.encode(v)

    from fused_turboquant import _lib
    L = _lib.lib()
    sp = _lib.stream_ptr(dev)
    signs, bnd, lev = tq.rotation.signs, tq.quantizer.boundaries, tq.quantizer.levels
    dec_out = torch.empty(T, H, d, dtype=torch.float32, device=dev)

    def enc_k():
        L.ftq_encode(k.data_ptr(), 2, n, d, signs.data_ptr(), bnd.data_ptr(), bits,
                     ck.indices.data_ptr(), ck.norms.data_ptr(), sp)

    def enc_v():
        L.ftq_encode(v.data_ptr(), 2, n, d, signs.data_ptr(), bnd.data_ptr(), bits,
                     cv.indices.data_ptr(), cv.norms.data_ptr(), sp)

    def dec_k():
        L.ftq_decode(ck.indices.data_ptr(), ck.norms.data_ptr(), n, d, lev.data_ptr(),
                     signs.data_ptr(), bits, dec_out.data_ptr(), 0, sp)

    attn = None
    try:
        from fused_turboquant import paged as P
        attn = P.bench_setup(dev)
    except (ImportError, AttributeError):
        attn = None

    def step():
        enc_k()
        enc_v()
        if attn is not None:
            attn["run"]()

    if args.calib_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_step = e0.elapsed_time(e1) / args.steps
    log(f"[bench] {args.steps} steps: {ms_step * 1e3:.1f} us/step (event), {wall_ms * 1e3:.1f} us/step (wall)")

    # per-kernel averages on the launch stream
    it = max(args.steps, 20)
    t_enc = time_launches(enc_k, it, torch)
    t_dec = time_launches(dec_k, it, torch)
    enc_bytes = n * d * 2 + n * (d * bits // 8) + n * 2
    dec_bytes = n * (d * bits // 8) + n * 2 + n * d * 4
    enc_in_gbs = n * d * 2 / (t_enc * 1e-6) / 1e9
    enc_gbs = enc_bytes / (t_enc * 1e-6) / 1e9
    dec_gbs = dec_bytes / (t_dec * 1e-6) / 1e9
    log(f"[bench] encode {t_enc:.2f} us  {enc_gbs:.0f} GB/s total ({enc_in_gbs:.0f} GB/s bf16 in)")
    log(f"[bench] decode {t_dec:.2f} us  {dec_gbs:.0f} GB/s total")

    extra = {}
    if attn is not None:
        t_attn = time_launches(attn["run"], it, torch)
        kv = attn["kv_bytes"]
        tot = attn["total_bytes"]
        extra["attn_us_per_step"] = round(t_attn, 2)
        extra["attn_kv_gbs"] = round(kv / (t_attn * 1e-6) / 1e9, 1)
        extra["attn_frac_hbm"] = round(tot / (t_attn * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        for kname, t in attn.get("kernels", {}).items():
            extra[f"attn_{kname}_us"] = round(time_launches(t, it, torch), 2)
        log(f"[bench] paged decode attention {t_attn:.2f} us/step, {extra['attn_kv_gbs']} GB/s KV")

    extra["decode_us"] = round(t_dec, 2)
    extra["decode_frac_hbm"] = round(dec_gbs / HBM_PEAK_GBS, 4)

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle encode on host cores)")
        cv_gbs, sample = cpu_baseline_encode()
        cpu = {"value": round(cv_gbs, 4), "unit": "GB/s (bf16 in)", "cores": 1, "kind": "port",
               "sample": sample + f"; host {platform.processor() or platform.machine()}, "
                                  f"os.cpu_count()={os.cpu_count()}, numpy single thread"}

    out = {
        "metric": "3-bit d128 encode GB/s + paged decode-attn us/step @8K ctx; % of HBM peak",
        "value": round(enc_in_gbs, 1),
        "unit": "GB/s (bf16 input consumed, 3-bit d=128 encode)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 in / fp32 math / u8 codes", "data": "synthetic",
        "config": {"workload": "config2 encode K+V [32768,8,128] bf16 3-bit"
                               + (" + config3 paged decode attention B=32 Hq=32 Hkv=8 ctx=8192 page=16"
                                  if attn is not None else ""),
                   "encode_us": round(t_enc, 2)},
        "roofline": {"bound": "hbm", "achieved": round(enc_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(enc_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "encode_kernel<128,3,bf16>", "algorithmic_bytes": enc_bytes},
        "cpu_baseline": cpu,
    }
    out.update(extra)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the MI355X fused-turboquant KV-cache hot path (one GPU).

One step = the BASELINE headline workload on one GPU, inputs resident in HBM:
  * config 2: fused 3-bit encode of K and of V, each [32768, 8, 128] bf16
    (262 144 vectors per tensor), TurboQuantMSE(128, bits=3, seed=42);
  * config 3: one paged decode-attention step over the 3-bit compressed
    library-format cache (B=32, Hq=32, Hkv=8, d=128, ctx 8192, page 16).
``value`` is the encode throughput in GB/s of bf16 input consumed.

Also timed (not part of the step): the d=256 encode and the d=128 decode of
config 2, config 4 (vLLM v1 slot format, K4V2, v_rotate, B=4, contexts
U[65536, 131072]) and the boundary-layer raw fp16 decode attention at the
config-3 shape (512-byte K|V slots, 1.07 GB).  Every kernel gets a roofline entry: algorithmic bytes per
launch / launch time, from HIP events on the stream the library launches on
(torch's current stream), in steady state: 20 untimed launches, then the
median of three windows of back-to-back launches.

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

# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this
# script, each scaled by the factor a 256 MiB device-to-device copy reads
# (FETCH x2.0, WRITE x1.0); the summaries are in profiles/hbm_traffic_counters.md.
# Keyed by roofline entry; None where no counter run covers the kernel.
TRAFFIC_BYTES: dict = {
    "encode_d128_3bit": 80336620, "encode_d256_3bit": 160154623, "decode_d128_3bit_f32": 149011545,
    "paged_attn_config3": 219810032, "v1_attn_config4": 406670855, "raw_attn_boundary": 1081506403,
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def time_launches(fn, iters, torch, warm=20, windows=3):
    """Device time of one fn() call in steady state, from HIP events on the
    current stream: `warm` untimed launches (clocks settle), then the median
    over `windows` windows of `iters` back-to-back launches."""
    st = torch.cuda.current_stream()
    for _ in range(warm):
        fn()
    per = []
    for _ in range(windows):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(iters):
            fn()
        e1.record(st)
        e1.synchronize()
        per.append(e0.elapsed_time(e1) * 1e3 / iters)  # us
    return sorted(per)[len(per) // 2]


def lean_launch(fn, keep, *args):
    """A C-ABI launch with its ctypes arguments converted once: host time per
    call stays well under a kernel's, so back-to-back launches leave no gaps.
    The arguments hold raw device pointers, so the tensors behind them (`keep`)
    stay referenced by the launcher.  Statuses are checked after the timed
    region (check_lean)."""
    import ctypes
    conv = tuple(ctypes.c_void_p(a) if isinstance(a, int) and abs(a) > 2 ** 40 else a for a in args)
    status = []

    def call():
        status.append(fn(*conv))
    call.status = status
    call.keep = tuple(keep)
    return call


def check_lean(*calls):
    from fused_turboquant import _lib
    for c in calls:
        for rc in c.status:
            _lib.check(rc)
        c.status.clear()


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


def roof(name, alg_bytes, t_us):
    gbs = alg_bytes / (t_us * 1e-6) / 1e9
    tr = TRAFFIC_BYTES.get(name)
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": tr, "kernel_us": round(t_us, 2),
            "algorithmic_bytes": alg_bytes}


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
    from fused_turboquant import TurboQuantMSE, _lib
    from fused_turboquant import paged as P
    from fused_turboquant import raw as R
    from fused_turboquant import v1 as V1

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = _lib.lib()
    sp = _lib.stream_ptr(dev)
    bits, T, H = 3, 32768, 8
    n = T * H

    def codec_setup(d, seed):
        g = torch.Generator(device="cpu").manual_seed(seed)
        sc = torch.exp(0.5 * torch.randn(d, generator=torch.Generator().manual_seed(seed + 1)))
        k = (torch.randn(T, H, d, generator=g) * sc).to(torch.bfloat16).to(dev)
        v = (torch.randn(T, H, d, generator=g) * sc).to(torch.bfloat16).to(dev)
        tq = TurboQuantMSE(d, bits=bits, seed=42, device=dev)
        ck, cv = tq.encode(k), tq.encode(v)
        signs, bnd = tq.rotation.signs, tq.quantizer.boundaries

        cls = tq.quantizer.codebook_class  # symmetric at d=128: the |t|-search kernel

        def enc(x, c):
            return lean_launch(L.ftq_encode_cb, (x, c, signs, bnd), x.data_ptr(), 2, n, d, signs.data_ptr(),
                               bnd.data_ptr(), bits, cls, c.indices.data_ptr(), c.norms.data_ptr(), sp)
        return tq, ck, enc(k, ck), enc(v, cv)

    log(f"[bench] config2 encode: [{T},{H},128] and [{T},{H},256] bf16 3-bit, K and V")
    tq128, ck128, enc_k, enc_v = codec_setup(128, 0)
    _, _, enc_k256, _ = codec_setup(256, 10)
    dec_out = torch.empty(T, H, 128, dtype=torch.float32, device=dev)
    lev, sg = tq128.quantizer.levels, tq128.rotation.signs

    dec_k = lean_launch(L.ftq_decode, (ck128, lev, sg, dec_out), ck128.indices.data_ptr(), ck128.norms.data_ptr(),
                        n, 128, lev.data_ptr(), sg.data_ptr(), bits, dec_out.data_ptr(), 0, sp)

    log("[bench] config3 paged cache (B=32 ctx=8192 K3V3)")
    attn3 = P.bench_setup(dev)
    log("[bench] config4 v1 cache (B=4 ctx~U[64K,128K] K4V2 v_rotate)")
    attn4 = V1.bench_setup(dev)
    log("[bench] boundary-layer raw fp16 cache (config3 shape, 512 B slots)")
    attnr = R.bench_setup(dev)
    torch.cuda.synchronize()

    def step():
        enc_k()
        enc_v()
        attn3["run"]()

    if args.calib_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    check_lean(enc_k, enc_v)
    t0 = time.perf_counter()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    check_lean(enc_k, enc_v)
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_step = e0.elapsed_time(e1) / args.steps
    log(f"[bench] {args.steps} steps: {ms_step * 1e3:.1f} us/step (event), {wall_ms * 1e3:.1f} us/step (wall)")

    it = max(args.steps, 20)
    t_enc = time_launches(enc_k, it, torch)
    t_enc256 = time_launches(enc_k256, it, torch)
    t_dec = time_launches(dec_k, it, torch)
    t_a3 = time_launches(attn3["run"], it, torch)
    t_a4 = time_launches(attn4["run"], it, torch)
    t_ar = time_launches(attnr["run"], it, torch)
    check_lean(enc_k, enc_k256, dec_k)

    enc_bytes = n * 128 * 2 + n * (128 * bits // 8) + n * 2
    enc256_bytes = n * 256 * 2 + n * (256 * bits // 8) + n * 2
    dec_bytes = n * (128 * bits // 8) + n * 2 + n * 128 * 4
    rl = {
        "encode_d128_3bit": roof("encode_d128_3bit", enc_bytes, t_enc),
        "encode_d256_3bit": roof("encode_d256_3bit", enc256_bytes, t_enc256),
        "decode_d128_3bit_f32": roof("decode_d128_3bit_f32", dec_bytes, t_dec),
        "paged_attn_config3": roof("paged_attn_config3", attn3["total_bytes"], t_a3),
        "v1_attn_config4": roof("v1_attn_config4", attn4["total_bytes"], t_a4),
        "raw_attn_boundary": roof("raw_attn_boundary", attnr["total_bytes"], t_ar),
    }
    for k, r in rl.items():
        log(f"[bench] {k}: {r['kernel_us']} us  {r['achieved']} GB/s  frac {r['frac']}")
    enc_in_gbs = n * 128 * 2 / (t_enc * 1e-6) / 1e9

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle encode on host cores)")
        cv_gbs, sample = cpu_baseline_encode()
        cpu = {"value": round(cv_gbs, 4), "unit": "GB/s (bf16 in)", "cores": 1, "kind": "port",
               "sample": sample + f"; host {platform.processor() or platform.machine()}, "
                                  f"os.cpu_count()={os.cpu_count()}, numpy single thread"}

    main_roof = dict(rl["encode_d128_3bit"])
    main_roof["kernel"] = "ftq::encode_mfma_kernel<128,3,bf16,sym>"
    out = {
        "metric": "3-bit d128 encode GB/s + paged decode-attn us/step @8K ctx; % of HBM peak",
        "value": round(enc_in_gbs, 1),
        "unit": "GB/s (bf16 input consumed, 3-bit d=128 encode)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 in / fp32 math / u8 codes", "data": "synthetic",
        "config": {"workload": "config2 encode K+V [32768,8,128] bf16 3-bit + config3 paged decode "
                               "attention B=32 Hq=32 Hkv=8 d=128 ctx=8192 page=16 K3V3",
                   "encode_us": round(t_enc, 2),
                   "attn_us_per_step": round(t_a3, 2),
                   "attn_kv_gbs": round(attn3["kv_bytes"] / (t_a3 * 1e-6) / 1e9, 1),
                   "attn_splits": attn3["splits"],
                   "config4_attn_us_per_step": round(t_a4, 2),
                   "config4_kv_gbs": round(attn4["kv_bytes"] / (t_a4 * 1e-6) / 1e9, 1),
                   "config4_ctx": attn4["lens"], "config4_splits": attn4["splits"]},
        "roofline": main_roof,
        "rooflines": rl,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

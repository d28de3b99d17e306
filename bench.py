"""Benchmark of the MI355X SageAttention path on BASELINE.json's metric configuration.

Workload: config 2, Flux-style joint attention, HND bf16 [1, 24, 4608, 128], non-causal, seeded synthetic inputs
(K with outlier channels), resident in HBM before the timed region.  One step = one ``sageattention.sageattn`` call,
i.e. the whole hot path: V amax, Q quantizer, K/V quantizer and the int8/fp8 attention kernel.

Prints ONE JSON line on stdout:
  value        whole-call throughput in TOPS (algorithmic ops 4*B*H*Sq*Skv*D per call / wall time per call)
  roofline     the attention kernel (dominant): achieved TFLOP/s from HIP events around back-to-back launches on the
               launch stream, against MI355X's dense int8/fp8 MFMA peak (5.0 PFLOP/s)
  cpu_baseline the reference's quantized math (the numpy port in oracle/) timed on this host on a head sample
Everything else (per-kernel times, quantizer GB/s, torch SDPA bf16 on the same GPU) goes to the "detail" object.

usage: python bench.py [--gpus 1] [--steps 100] [--warmup 20] [--no-cpu-baseline] [--config 2]
       python bench.py --models [name ...]      (the reference's model-shape table; one JSON line with every row)

--config takes a configuration of cdna4_sage.configs: 2 (default), 3, 4, 5a, 5b, 1, lumina (head dim 96),
auraflow (head dim 256).

Order: 0.3 s of forward calls take the GPU clock out of its idle state (in which the first ~25 ms of calls run ~15%
slower), then the per-kernel measurements run, then exactly --warmup untimed steps and the --steps timed ones (mean
time per call, back to back).  detail.median_synced_ms adds the reference's method (tests/bench_models.py:45-53:
3 warm-up calls, then the median of 10 calls each followed by a synchronisation).  The torch SDPA and masked-call
comparisons run last: right after 100 SDPA calls the sageattn call runs ~1.4% slower, recovering over the next ~200
calls (196.1 -> 198.8 -> 196.3 us on one MI355X).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT / "rdna4-sageattention_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

MFMA_PEAK_TFLOPS = 5000.0   # MI355X dense int8 / OCP-fp8 MFMA, ops/s / 1e12
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_events(fn, iters):
    """Average ms per call of fn() launched back to back on torch's current stream, measured with HIP events."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def cpu_baseline(cfg, target_s=15.0):
    """Time the numpy port of the reference's quantized math on a sample of whole heads (full sequence), as many
    heads as fit ~target_s of work; report TOPS of the sample.  Also time torch SDPA fp32 on the CPU per head."""
    import numpy as np
    import torch

    from cdna4_sage.configs import make_inputs
    from oracle import sage_oracle as orc

    threads = torch.get_num_threads()
    grp = cfg.H // cfg.Hkv

    def one(nh):
        q, k, v = make_inputs(cfg, heads=slice(0, nh))
        qn, kn, vn = (t.float().numpy() for t in (q, k, v))
        t0 = time.perf_counter()
        q8, qs = orc.quant_q(qn)
        k8, ks, v8, vs = orc.quant_kv(kn, vn)
        orc.attention(q8, qs, k8, ks, v8, vs, kn.shape[2], causal=cfg.causal, block_n=32)
        return time.perf_counter() - t0, (q, k, v)

    t1, _ = one(1)                                   # one kv head (and its query heads) to size the sample
    nh = int(max(1, min(cfg.Hkv, target_s // max(t1, 1e-3))))
    if nh > 1:
        t_emu, (q, k, v) = one(nh)
    else:
        t_emu, (q, k, v) = t1, make_inputs(cfg, heads=slice(0, 1))
    ops = cfg.attention_ops() * nh / cfg.Hkv
    # torch SDPA fp32 on the CPU, same heads
    qf, kf, vf = (t.float() for t in (q, k, v))
    t0 = time.perf_counter()
    torch.nn.functional.scaled_dot_product_attention(qf, kf.repeat_interleave(grp, 1), vf.repeat_interleave(grp, 1),
                                                     is_causal=cfg.causal)
    t_sdpa = time.perf_counter() - t0
    return {
        "value": round(ops / t_emu / 1e12, 6),
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"{nh * grp} of {cfg.H} query heads ({nh} kv heads) of {cfg.name}, full sequence; numpy float32 "
                  f"emulation of the quantized path (block_n 32), {t_emu:.2f} s; whole call extrapolated "
                  f"x{cfg.Hkv / nh:.1f} = {t_emu * cfg.Hkv / nh * 1e3:.0f} ms",
        "sdpa_fp32_cpu_tops": round(ops / t_sdpa / 1e12, 6),
        "sdpa_fp32_cpu_ms_extrapolated": round(t_sdpa * cfg.Hkv / nh * 1e3, 1),
        "host_cpus": os.cpu_count(),
    }


PROFILE_STEMS = {"2": "flux_config2", "3": "wan14b_config3", "4": "hunyuan_config4", "5a": "causal_gqa_config5a",
                 "5b": "causal_gqa_d64_config5b", "lumina": "neta_lumina_d96", "auraflow": "auraflow_d256"}

def intermediates(cfg, dev):
    """Q8, QS, K8, KS, V8T, VS of one sage_forward call on cfg, in the C ABI's layouts (include/sage_capi.h): the
    int8 / E4M3 rows have sage_layout_dim(D) channels (128 for head dim 96, zero-padded), the key axis
    sage_kv_pad(S) rows."""
    import torch

    from cdna4_sage import _capi

    B, H, Hkv, S, D = cfg.B, cfg.H, cfg.Hkv, cfg.S, cfg.D
    skp, dl = _capi.kv_pad(S), _capi.layout_dim(D)
    return (torch.empty(B, H, S, dl, dtype=torch.int8, device=dev),
            torch.empty(B, H, S, dtype=torch.float32, device=dev),
            torch.empty(B, Hkv, skp, dl, dtype=torch.int8, device=dev),
            torch.empty(B, Hkv, skp // 32, dtype=torch.float32, device=dev),
            torch.empty(B, Hkv, dl, skp, dtype=torch.uint8, device=dev),
            torch.empty(B, Hkv, dl, dtype=torch.float32, device=dev))


def median_synced_ms(fn, n=10):
    """The reference's per-call time: 3 warm-up calls, then the median of n calls each followed by a sync."""
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(n):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(ts)


def bench_models(only):
    """Every shape of MODEL_SHAPES (or those whose name contains one of `only`): SDPA, kernel-forced and routed
    ms per call, and the kernel's TOPS (4 * B * H * pairs * D per call, pairs = Sq * Skv or its causal half)."""
    import torch
    import torch.nn.functional as F

    import cdna4_sage
    import sageattention
    from cdna4_sage.configs import MODEL_SHAPES

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    dts = {"bf16": torch.bfloat16, "f16": torch.float16}
    rows = []
    log(f"{'shape':26s} {'sdpa ms':>9s} {'kernel ms':>10s} {'speedup':>8s} {'routed ms':>10s} {'TOPS':>7s}  route")
    for name, B, Sq, Skv, H, D, layout, dt, causal in MODEL_SHAPES:
        if only and not any(o.lower() in name.lower() for o in only):
            continue
        g = torch.Generator().manual_seed(len(rows))
        shp = (lambda s: (B, H, s, D)) if layout == "HND" else (lambda s: (B, s, H, D))  # noqa: E731
        q, k, v = (torch.randn(shp(s), generator=g).to(dts[dt]).to(dev) for s in (Sq, Skv, Skv))
        hnd = (lambda x: x) if layout == "HND" else (lambda x: x.transpose(1, 2))  # noqa: E731
        t_sdpa = median_synced_ms(lambda: F.scaled_dot_product_attention(hnd(q), hnd(k), hnd(v), is_causal=causal))
        try:
            t_kern = median_synced_ms(lambda: cdna4_sage.attention(q, k, v, layout, is_causal=causal))
        except cdna4_sage.Unsupported:
            t_kern = None
        t_route = median_synced_ms(lambda: sageattention.sageattn(q, k, v, tensor_layout=layout, is_causal=causal))
        routed = t_kern is not None and cdna4_sage._worth_it(q, k, layout, causal)
        pairs = Sq * (Sq + 1) // 2 if causal and Sq == Skv else Sq * Skv
        tops = 4 * B * H * pairs * D / (t_kern * 1e-3) / 1e12 if t_kern else None
        row = {"shape": name, "B": B, "Sq": Sq, "Skv": Skv, "H": H, "D": D, "layout": layout, "dtype": dt,
               "causal": causal, "sdpa_ms": round(t_sdpa, 4), "kernel_ms": None if t_kern is None else round(t_kern, 4),
               "speedup": None if t_kern is None else round(t_sdpa / t_kern, 3), "routed_ms": round(t_route, 4),
               "kernel_TOPS": None if tops is None else round(tops, 1), "route": "kernel" if routed else "sdpa"}
        rows.append(row)
        log(f"{name:26s} {t_sdpa:9.3f} {t_kern if t_kern else float('nan'):10.3f} "
            f"{(t_sdpa / t_kern) if t_kern else float('nan'):7.2f}x {t_route:10.3f} {tops or float('nan'):7.1f}  "
            f"{row['route']}")
        del q, k, v
        torch.cuda.empty_cache()
    print(json.dumps({"metric": "per-call ms of the reference's model shapes (tests/bench_models.py), SDPA vs "
                                "kernel vs routed", "unit": "ms", "higher_is_better": False, "n_gpus": 1,
                      "method": "median of 10 synced calls after 3 warm-ups", "data": "synthetic N(0,1)",
                      "device": torch.cuda.get_device_name(dev), "shapes": rows}), flush=True)


def profiled_traffic(cfg_key):
    """HBM bytes per attention call (attention kernel + merge of split tiles) from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of this configuration."""
    stem = PROFILE_STEMS.get(cfg_key)
    f = ROOT / "profiles" / f"{stem}_profile.md" if stem else None
    if f is None or not f.exists():
        return None, None
    for line in f.read_text().splitlines():
        if line.startswith("attention traffic_bytes_per_call:"):
            return int(line.split(":")[1]), str(f.relative_to(ROOT))
    return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20, help="untimed steps right before the timed ones")
    ap.add_argument("--config", default="2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-iters", type=int, default=50)
    ap.add_argument("--compare-unsplit", action="store_true",
                    help="also time the attention with every query tile whole (no workspace)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run one plain device copy of this many MiB first (calibrates rocprofv3 FETCH/WRITE_SIZE)")
    ap.add_argument("--models", nargs="*", default=None,
                    help="time the reference's model shapes instead (all, or those whose name contains an argument)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} is not supported (each call is a single-device "
              "op on one GPU; sharding heads or sequences over several GPUs is not built)", file=sys.stderr)
        sys.exit(2)
    if args.models is not None:
        bench_models(args.models)
        return

    import torch
    import torch.nn.functional as F

    import cdna4_sage
    import sageattention
    from cdna4_sage import _attention, _capi
    from cdna4_sage.configs import CONFIGS, make_inputs

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_probe_mib > 0:
        src = torch.ones(args.copy_probe_mib * 2**20 // 4, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log(f"device {torch.cuda.get_device_name(dev)} arch {_attention.device_arch(dev)}; workload {cfg.name}")
    q, k, v = (t.to(dev) for t in make_inputs(cfg))
    torch.cuda.synchronize()

    routed = cdna4_sage._worth_it(q, k, "HND", cfg.causal)
    if routed:
        def step():
            return sageattention.sageattn(q, k, v, tensor_layout="HND", is_causal=cfg.causal,
                                          return_lse=cfg.return_lse)
    else:
        # below the router's minimum size sageattn uses SDPA, as the reference does: time the kernel-forced entry
        def step():
            return cdna4_sage.attention(q, k, v, "HND", is_causal=cfg.causal)
    ops = cfg.attention_ops()

    # ---- per-kernel times: the same launches the call makes, each looped on torch's current stream ----
    B, H, Hkv, S, D = cfg.B, cfg.H, cfg.Hkv, cfg.S, cfg.D
    skp = _capi.kv_pad(S)
    st = torch.cuda.current_stream(dev).cuda_stream
    q8, qs, k8, ks, v8t, vs = intermediates(cfg, dev)
    out = torch.empty(B, S, H, D, dtype=q.dtype, device=dev)
    hs = (q.stride(0), q.stride(2), q.stride(1))
    ks_ = (k.stride(0), k.stride(2), k.stride(1))
    vs_ = (v.stride(0), v.stride(2), v.stride(1))
    dt = _capi.DTYPE_BF16 if q.dtype == torch.bfloat16 else _capi.DTYPE_F16
    L = _capi.lib()

    # the C forward call exactly as the step makes it (two quantization launches, attention, merge of split tiles)
    fws = _capi.forward_workspace(0, B, H, Hkv, S, S, D, cfg.causal)
    fwbuf = torch.empty(max(fws, 1), dtype=torch.uint8, device=dev)

    def k_forward():
        L.sage_forward(q.data_ptr(), *hs, k.data_ptr(), *ks_, v.data_ptr(), *vs_, out.data_ptr(), out.stride(0),
                       out.stride(1), out.stride(2), B, H, Hkv, S, S, D, dt, int(cfg.causal), 1.0, q8.data_ptr(),
                       qs.data_ptr(), k8.data_ptr(), ks.data_ptr(), v8t.data_ptr(), vs.data_ptr(), fwbuf.data_ptr(),
                       fws, st)

    # the attention launch(es) alone, on the intermediates the forward call left
    n_full, chunks, ws_bytes = _capi.attn_plan(0, B, H, S, S, D, cfg.causal)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

    def k_attn(split=True):
        L.sage_attn_fwd(q8.data_ptr(), qs.data_ptr(), k8.data_ptr(), ks.data_ptr(), v8t.data_ptr(), vs.data_ptr(),
                        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), B, H, Hkv, S, S, D,
                        int(cfg.causal), dt, None, ws.data_ptr() if split and ws_bytes else None,
                        ws_bytes if split else 0, st)

    # the GPU clock leaves its idle state within ~25 ms of busy calls: spin the forward for 0.3 s before any timing
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.3:
        for _ in range(10):
            k_forward()
        torch.cuda.synchronize()
    it = args.kernel_iters
    t_fwd = time_events(k_forward, it)
    t_attn = time_events(k_attn, it)
    t_attn_whole = time_events(lambda: k_attn(False), it) if args.compare_unsplit else None
    attn_tflops = ops / (t_attn * 1e-3) / 1e12
    quant_bytes = cfg.quant_q_bytes() + cfg.quant_kv_bytes(skp)

    # ---- the step: exactly --warmup untimed calls, then --steps timed calls back to back ----
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    tops = ops / (ms * 1e-3) / 1e12
    # the reference's method (tests/bench_models.py:45-53): 3 warm-ups, median of 10 synchronised calls
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    synced = []
    for _ in range(10):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        synced.append((time.perf_counter() - t0) * 1e3)
    ms_median_synced = statistics.median(synced)

    # ---- torch SDPA bf16 on the same GPU, same method as the step ----
    sdpa = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=cfg.causal, enable_gqa=Hkv != H)  # noqa: E731
    for _ in range(20):
        sdpa()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        sdpa()
    torch.cuda.synchronize()
    ms_sdpa = (time.perf_counter() - t0) * 1e3 / args.steps

    # ---- a boolean key-padding mask (the last eighth of the keys hidden): the masked call, timed like the step, and
    # torch SDPA bf16 with the same mask (non-causal configurations) ----
    masked = None
    if not cfg.causal:
        mask = (torch.arange(S, device=dev) < S - S // 8)[None, None, None, :].expand(B, 1, 1, S)

        def wall(fn, n):
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(n):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / n

        if routed:
            mfn = lambda: sageattention.sageattn(q, k, v, tensor_layout="HND", attn_mask=mask)  # noqa: E731
        else:
            mfn = lambda: cdna4_sage.attention(q, k, v, "HND", attn_mask=mask)  # noqa: E731
        ms_mask = wall(mfn, args.steps)
        ms_mask_sdpa = wall(lambda: F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=Hkv != H),
                            max(10, args.steps // 10))
        masked = {"mask": f"bool [B, 1, 1, S], first {S - S // 8} of {S} keys visible", "ms": round(ms_mask, 4),
                  "sdpa_bf16_ms": round(ms_mask_sdpa, 4), "speedup_vs_sdpa_bf16": round(ms_mask_sdpa / ms_mask, 3)}

    traffic, traffic_src = profiled_traffic(args.config)
    result = {
        "metric": "attention TOPS + ms/call (Flux 24x4608x128), % of int8/fp8 MFMA peak",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 QK / fp8-e4m3 PV (fp32 softmax, bf16 in/out)",
        "data": "synthetic (seeded, CPU-generated, resident in HBM)",
        "config": {"workload": cfg.name, "B": B, "H": H, "Hkv": Hkv, "Sq": S, "Skv": S, "D": D,
                   "layout": "HND", "input_dtype": str(q.dtype).replace("torch.", ""), "causal": cfg.causal},
        "roofline": {"bound": "mfma", "achieved": round(attn_tflops, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(attn_tflops / MFMA_PEAK_TFLOPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": f"attn_kernel<{D},{str(cfg.causal).lower()},bf16>"
                               + (" + attn_merge_kernel" if chunks > 1 else ""),
                     "ms_per_launch": round(t_attn, 5), "ops_per_launch": ops,
                     "plan": {"whole_tiles": n_full, "split_tiles": B * H * ((S + 127) // 128) - n_full,
                              "kv_chunks": chunks, "workspace_bytes": ws_bytes}},
        "detail": {
            "step": "sageattention.sageattn" if routed else "cdna4_sage.attention (sageattn routes this size to SDPA)",
            "call_frac_of_peak": round(tops / MFMA_PEAK_TFLOPS, 4),
            "median_synced_ms": round(ms_median_synced, 4),
            "kernel_ms": {"forward_capi": round(t_fwd, 5), "attn": round(t_attn, 5),
                          "quant (forward - attn)": round(t_fwd - t_attn, 5)},
            "quant_GBps": round(quant_bytes / ((t_fwd - t_attn) * 1e-3) / 1e9, 1),
            "hbm_peak_GBps": HBM_PEAK_GBS,
            "sdpa_bf16_gpu_ms": round(ms_sdpa, 4),
            "speedup_vs_sdpa_bf16": round(ms_sdpa / ms, 3),
            "device": torch.cuda.get_device_name(dev),
        },
    }
    if masked is not None:
        result["detail"]["key_padding_mask"] = masked
    if t_attn_whole is not None:
        result["detail"]["kernel_ms"]["attn_without_split"] = round(t_attn_whole, 5)
    if cfg.return_lse:
        # the LSE the step returns, timed alone (bf16 MFMA kernel; 2 flops per multiply-add of Q K^T)
        t_lse = time_events(lambda: cdna4_sage.lse(q, k, "HND", None, cfg.causal), it)
        result["detail"]["kernel_ms"]["lse"] = round(t_lse, 5)
        result["detail"]["lse_bf16_TFLOPs"] = round(2 * B * H * cfg.pairs() * D / (t_lse * 1e-3) / 1e12, 1)
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(cfg)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Batch-1 greedy decode throughput of the 7B-shape Q4_0 model on one MI355X.

A step is one decoded token: the full forward pass (32 layers, untied Q4_0 LM
head) plus the device argmax feeding the next step, after a 512-token prefill.
Inside the timed steps every 8th weight-GEMV dispatch records start/stop HIP
events as part of the dispatch (on its stream). Per projection (the launches
split by the weight bytes they stream) their average duration gives achieved
GB/s against the 8 TB/s HBM peak; the roofline object is the projection with
the most time per token. The Q|K|V and gate|up launches also compute their
input's rmsnorm (one fewer launch each), so their duration includes it. The same number of steps is also
timed without any events (reported beside). The
HBM traffic per GEMV launch comes from the committed rocprofv3 counter
summary (profiles/q4_0_gemv_7b_decode_traffic.json) when present. The
reference's CPU path is timed on a bounded sample of the same workload: its
scalar tier (the parity oracle, whose greedy stream the GPU must reproduce)
and its timed tier (runtime-selected SIMD dots on its persistent pool, at its
default min(nproc, 8) threads and at all host cores), both C restatements.

Prints one JSON line. --gpus above 1 is not supported by this build.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# prana_gemv_profile_shapes entry of the decode attention launch (no GEMV streams 1 byte)
ATTENTION_PROFILE_KEY = 1


def log(msg):
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


def host_info():
    """nproc, the CPU model name and the SIMD features the reference's runtime
    dispatch looks at (simd_x86.rs:18-29)."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name") and model == "unknown":
                    model = ln.split(":", 1)[1].strip()
                elif ln.startswith("flags") and not flags:
                    flags = set(ln.split(":", 1)[1].split())
    except OSError:
        pass
    simd = [x for x in ("avx2", "fma", "avx_vnni", "avx512_vnni", "avx512bw") if x in flags]
    return {"nproc": os.cpu_count(), "model": model, "simd": simd}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prefill", type=int, default=512)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 512 MiB device-to-device copy (the reference kernel for HBM counter scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the decode path would shard by weight rows and KV heads, which is not built.", file=sys.stderr)
        sys.exit(2)

    import prana_amd as P
    from prana_amd import models as M

    cfg = dict(M.C4)
    K, W, npre = args.steps, args.warmup, args.prefill
    t0 = time.time()
    tensors = M.synth_tensors(cfg, M.types_c4, 4)
    log(f"synthesized {sum(v[2].nbytes for v in tensors.values()) / 1e9:.2f} GB of weights in {time.time() - t0:.1f}s")
    t0 = time.time()
    model = P.Model(cfg, tensors)
    stream_bytes = model.stream_bytes()
    log(f"uploaded model in {time.time() - t0:.1f}s; {stream_bytes / 1e9:.4f} GB of weights streamed per token")

    if args.copy_calibration:
        nb = 512 << 20
        a, b = P.DeviceArray(nb, np.uint8), P.DeviceArray(nb, np.uint8)
        P.check(P.load().prana_memset_d(a.ptr, 1, nb))
        P.check(P.load().prana_memcpy_d2d(b.ptr, a.ptr, nb))
        a.free()
        b.free()
        log(f"calibration copy: {nb} bytes device to device")

    rng = np.random.default_rng(512)
    prompt = rng.integers(0, cfg["vocab_size"], npre).astype(np.uint32)
    cache = model.cache(npre + W + 2 * K + 2)
    t0 = time.perf_counter()
    cache.prefill(prompt[:-1])
    prefill_s = time.perf_counter() - t0
    log(f"prefill {npre - 1} tokens: {prefill_s:.3f}s")

    pos = npre - 1
    toks = cache.decode(int(prompt[-1]), pos, W)
    pos += W
    last = int(toks[-1]) if W else int(prompt[-1])
    log(f"warmup {W} steps done")

    # Timed region: K decode steps. Every 8th weight-GEMV dispatch carries
    # start/stop HIP events (dispatch timestamps on its stream); 129 GEMV
    # launches per token make the sampled launches rotate over all shapes.
    P.gemv_profile(True, period=8)
    P.gemv_profile_read(reset=True)
    P.check(P.load().prana_synchronize())
    t0 = time.perf_counter()
    toks = cache.decode(last, pos, K)
    P.check(P.load().prana_synchronize())
    dt = time.perf_counter() - t0
    shapes = P.gemv_profile_shapes()
    n_launch, gsec, gbytes = P.gemv_profile_read(reset=True)
    P.gemv_profile(False)
    pos += K
    tok_s = K / dt
    gemv_gbs = gbytes / gsec / 1e9 if gsec > 0 else 0.0
    log(f"timed {K} decode steps: {dt * 1e3:.2f} ms -> {tok_s:.1f} tok/s")
    log(f"GEMV: {n_launch} timed launches, avg {gsec / max(n_launch, 1) * 1e6:.2f} us, {gemv_gbs:.1f} GB/s")

    # The same number of steps again without any events.
    P.check(P.load().prana_synchronize())
    t0 = time.perf_counter()
    cache.decode(int(toks[-1]), pos, K)
    P.check(P.load().prana_synchronize())
    dt_plain = time.perf_counter() - t0
    log(f"run without events: {K / dt_plain:.1f} tok/s")

    # the projections by the Q4_0 bytes they stream (18 bytes per 32 weights)
    d, hid, kv, voc = cfg["dim"], cfg["hidden_dim"], cfg["n_kv_heads"] * cfg["head_dim"], cfg["vocab_size"]
    q4 = lambda rows, cols: rows * cols // 32 * 18
    names = {q4(d + 2 * kv, d): ("Q|K|V + attention rmsnorm", cfg["n_layers"]),
             q4(d, d): ("wo", cfg["n_layers"]),
             2 * q4(hid, d): ("gate|up + SiLU + FFN rmsnorm", cfg["n_layers"]),
             q4(d, hid): ("down", cfg["n_layers"]),
             q4(voc, d): ("LM head", 1)}
    per, attn = [], None
    for b, n, sec in shapes:
        if b == ATTENTION_PROFILE_KEY:  # the one-launch decode attention kernel, sampled in the same rotation
            us = sec / max(n, 1) * 1e6
            attn = {"launches": n, "avg_us": round(us, 3), "per_token": cfg["n_layers"],
                    "us_per_token": round(us * cfg["n_layers"], 1)}
            continue
        name, per_tok = names.get(b, (f"{b} bytes", 0))
        us = sec / max(n, 1) * 1e6
        gbs = b / (sec / n) / 1e9 if sec > 0 else 0.0
        per.append({"name": name, "bytes": b, "launches": n, "avg_us": round(us, 3), "gbs": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4), "per_token": per_tok,
                    "us_per_token": round(us * per_tok, 1)})
    dom = max(per, key=lambda r: r["us_per_token"]) if per else None
    for r in per:
        log(f"  {r['name']:<30} {r['avg_us']:8.2f} us  {r['gbs']:8.1f} GB/s  ({r['frac'] * 100:.1f} %)")
    # A decode token split into sections: each projection's launches and the
    # attention launches (the norms run inside the Q|K|V and gate|up launches).
    # Dispatch-timestamp durations include each dispatch's start, which
    # back-to-back launches overlap, so their sum can exceed the token time.
    tok_us = dt_plain / K * 1e6
    sections = {r["name"]: r["us_per_token"] for r in per if r["per_token"]}
    if attn is not None:
        sections["attention (score, softmax, PV, wo input quantization)"] = attn["us_per_token"]
        log(f"  {'attention':<30} {attn['avg_us']:8.2f} us x {attn['per_token']} per token")
    decode_sections = {"token_us": round(tok_us, 1), "sampled_us_per_token": sections,
                       "sampled_sum_us": round(sum(sections.values()), 1)}
    log(f"per-token sections (us, token {tok_us:.1f}): " + ", ".join(f"{k}: {v}" for k, v in sections.items()))

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "q4_0_gemv_7b_decode_traffic.json")
    if os.path.exists(tpath) and dom is not None:
        with open(tpath) as f:
            t = json.load(f).get("hbm_bytes_per_launch")
        traffic = t.get(dom["name"]) if isinstance(t, dict) else None

    cpu, match = None, None
    if not args.no_cpu:
        from oracle import oracle as O
        threads = int(os.environ.get("PRANA_ORACLE_THREADS", min(16, os.cpu_count() or 1)))
        os.environ["PRANA_ORACLE_THREADS"] = str(threads)
        t0 = time.time()
        om = O.Model(cfg, tensors)
        log(f"oracle model built in {time.time() - t0:.1f}s")

        def cpu_decode(n_max, seconds):
            oc = om.cache(64)
            tok, toks, t0 = int(prompt[0]), [], time.perf_counter()
            while len(toks) < n_max and (len(toks) < 2 or time.perf_counter() - t0 < seconds):
                tok = int(O.argmax(oc.forward(tok, len(toks))))
                toks.append(tok)
            return toks, time.perf_counter() - t0

        # 1) the scalar tier (the parity oracle): the reference stream
        O.set_tier(0)
        cpu_toks, sdt = cpu_decode(60, args.cpu_seconds)
        n = len(cpu_toks)
        log(f"scalar tier: {n} steps, {n / sdt:.3f} tok/s on {threads} threads")
        # 2) the reference's timed tier (runtime-selected SIMD dots on its
        #    persistent pool) at its default thread count, then at all cores,
        #    over the same positions
        t_def = O.set_tier(1, 0)
        tier_toks, tdt = cpu_decode(n, 1e9)
        t_all = O.set_tier(1, os.cpu_count() or 1)
        _, adt = cpu_decode(n, 1e9)
        simd = O.tier_name()
        O.set_tier(0)
        log(f"timed tier [{simd}]: {n / tdt:.3f} tok/s on {t_def} threads, {n / adt:.3f} on {t_all}")
        cpu = {"value": round(n / tdt, 4), "unit": "tok/s", "cores": t_def, "kind": "port",
               "sample": f"{n} greedy decode steps of the same 7B-shape Q4_0 model at positions 0..{n - 1} from "
                         f"prompt id {int(prompt[0])}: the reference's timed tier (SIMD dots: {simd}; persistent "
                         f"spin-then-park pool of min(nproc, 8) = {t_def} threads), {tdt:.1f}s of CPU work",
               "all_cores": {"threads": t_all, "value": round(n / adt, 4)},
               "scalar_tier": {"threads": threads, "value": round(n / sdt, 4),
                               "note": "the oracle tier (pthreads per call), the parity reference"},
               "timed_tier_tokens_match_scalar": f"{sum(a == b for a, b in zip(tier_toks, cpu_toks))}/{n}",
               "host": host_info()}
        # The GPU decodes the very same steps (same prompt id, positions
        # 0..n-1, fresh cache); its stream must equal the scalar tier's.
        gcache = model.cache(n + 1)
        P.check(P.load().prana_synchronize())
        t0 = time.perf_counter()
        gpu_toks = [int(x) for x in gcache.decode(int(prompt[0]), 0, n)]
        P.check(P.load().prana_synchronize())
        gdt = time.perf_counter() - t0
        same = 0
        while same < n and gpu_toks[same] == cpu_toks[same]:
            same += 1
        match = {"tokens_match": f"{same}/{n}", "positions": f"0..{n - 1}",
                 "gpu_tok_s_same_positions": round(n / gdt, 3)}
        log(f"token streams: {same}/{n} identical (GPU {n / gdt:.1f} tok/s at the same positions)")

    line = {
        "metric": "batch-1 decode tok/s + weight-GEMV HBM GB/s (% of peak), 7B-shape Q4_0",
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(dt * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xQ4_0 dots (i32), f32 epilogues",
        "data": "synthetic (seeded N(0,0.02) random-init weights, random prompt ids)",
        "config": {
            "workload": "7B-shape llama (dim 4096, 32 layers, 32/8 heads, FFN 14336, vocab 32000), all Q4_0, "
                        f"untied Q4_0 head; greedy decode at batch 1 after a {npre}-token prefill",
            "prefill_tokens": npre,
            "weight_bytes_per_token": stream_bytes,
            "decode_weight_stream_gbs": round(stream_bytes * tok_s / 1e9, 2),
            "prefill_tok_s": round((npre - 1) / prefill_s, 2),
            "tok_s_without_events": round(K / dt_plain, 3),
            "decode_sections": decode_sections,
            "attention_launch": attn,
            "parity": match if match is not None else "not checked (--no-cpu)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": dom["gbs"] if dom else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dom["frac"] if dom else None,
            "traffic": traffic,
            "kernel": f"Q4_0 decode {dom['name']} (gemv_tile_kernel)" if dom else None,
            "timed_launches": dom["launches"] if dom else 0,
            "avg_launch_us": dom["avg_us"] if dom else None,
            "bytes_per_launch": dom["bytes"] if dom else None,
            "per_projection": per,
            "all_gemv_launches": {"timed_launches": n_launch,
                                  "avg_launch_us": round(gsec / max(n_launch, 1) * 1e6, 3),
                                  "gbs": round(gemv_gbs, 1), "frac": round(gemv_gbs / HBM_PEAK_GBS, 4)},
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    if match is not None and match["tokens_match"].split("/")[0] != match["tokens_match"].split("/")[1]:
        log("FAIL: the GPU token stream differs from the CPU reference path")
        sys.exit(1)


if __name__ == "__main__":
    main()

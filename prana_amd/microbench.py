#!/usr/bin/env python3
"""Kernel microbenchmarks for the configurations beside the headline decode.

C1: the Q8_0 matmul sweep (R x K in {4096x4096, 14336x4096, 4096x14336,
32000x4096}, N in {1, 4, 16, 64} tokens). Weight copies rotate so that the
bytes touched per case exceed twice the 256 MB MALL.
GEMM: the batched matrix-core GEMMs at the prefill batches of C4 (N = 511:
Q4_0 Q|K|V, wo, gate, down) and C2 (N = 2047: Q6_K ffn_down, a Q4_K
4096-column matrix, Q4_0 / Q8_0 896-column matrices), plus C1's Q8_0
4096x4096 at N = 16 and 64 (the skinny kernel), over pre-quantized
activations, reported as int8 TOPS against the 5.0 POPS dense peak.
C3: attention over an f16 cache (32 query / 8 KV heads, head_dim 128) at
contexts 1024, 4096, 16384 and 32768, q and the new k row under NeoX RoPE at
position = context: one sequence (decode) on the exact kernels and on split-K
flash decoding, eight query rows over one cache (the verify form), and batch
8 as eight independent caches on both paths. Cache copies rotate so that the
bytes touched per case exceed twice the MALL.

Timing comes from a rocprofv3 kernel trace, so there is no host overhead in
the figures. Run

    rocprofv3 --kernel-trace -d OUT -o run -- python3 -m prana_amd.microbench
    python3 -m prana_amd.microbench --summarize OUT/.../run_results.db

The run writes a case manifest (JSON). In the trace, each case is bracketed
by small fill-kernel markers: one before its warmup calls, one before its
timed calls and one after them, so set-up work (uploads, repacking) never
lands in a timed group. The summary sums every non-runtime kernel between
the second and third marker of a case, activation quantization included.
"""
import argparse
import ctypes as C
import json
import os
import sqlite3
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

Q8_0 = 8
MALL = 256 << 20
C1_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (32000, 4096)]
C1_TOKENS = [1, 4, 16, 64]
C3_CTX = [1024, 4096, 16384, 32768]
ATTN_ROWS = [545, 640, 1024]  # decode attention at the 7B bench's cache lengths (512-token prefill + steps)
WARMUP, TIMED = 3, 20
Q4_0, Q4_K, Q6_K = 2, 12, 14
GEMM_CASES = [  # (tag, ggml type, rows, cols, N)
    ("C4 Q|K|V Q4_0", Q4_0, 6144, 4096, 511), ("C4 wo Q4_0", Q4_0, 4096, 4096, 511),
    ("C4 ffn_gate Q4_0", Q4_0, 14336, 4096, 511), ("C4 ffn_down Q4_0", Q4_0, 4096, 14336, 511),
    ("C2 ffn_down Q6_K", Q6_K, 896, 4864, 2047), ("C2-width Q4_K", Q4_K, 512, 4096, 2047),
    ("C2 ffn_gate Q4_0", Q4_0, 4864, 896, 2047), ("C2 attn_v Q8_0", Q8_0, 128, 896, 2047),
    ("C1 Q8_0", Q8_0, 4096, 4096, 16), ("C1 Q8_0", Q8_0, 4096, 4096, 64),
]


VERIFY_SHAPES = [("Q|K|V", 6144, 4096), ("wo", 4096, 4096), ("ffn_down", 4096, 14336), ("head", 32000, 4096)]
VERIFY_TOKENS = [2, 5, 9, 16]


def _marker(P, buf):
    P.check(P.load().prana_memset_d(buf.ptr, 0, 256))


def run(manifest_path, only=None):
    import prana_amd as P

    P.init()
    marker = P.DeviceArray((256,), np.uint8)
    cases = []
    rng = np.random.default_rng(0)

    for rows, cols in (C1_SHAPES if only in (None, "C1") else []):
        raw = P.synth_tensor(Q8_0, rows, cols, rows * 7 + cols, 0.02)
        copies = max(3, -(-2 * MALL // raw.nbytes))
        mats = [P.Matrix(Q8_0, rows, cols, raw) for _ in range(copies)]
        print(f"C1 Q8_0 {rows}x{cols}: {copies} copies", file=sys.stderr, flush=True)
        for n in C1_TOKENS:
            x = P.DeviceArray.from_host(rng.standard_normal((n, cols)).astype(np.float32))
            out = P.DeviceArray((n, rows), np.float32)
            for phase, calls in (("warmup", WARMUP), ("timed", TIMED)):
                _marker(P, marker)
                for i in range(calls):
                    P.check(P.load().prana_matmul(mats[i % copies].h, x.ptr, n, out.ptr, None))
            _marker(P, marker)
            P.check(P.load().prana_synchronize())
            cases.append({"config": "C1", "case": f"Q8_0 {rows}x{cols} N={n}", "calls": TIMED,
                          "bytes": rows * cols // 32 * 34 + n * cols * 4 + n * rows * 4, "copies": copies})
        del mats

    for tag, ty, rows, cols, n in (GEMM_CASES if only in (None, "GEMM") else []):
        raw = P.synth_tensor(ty, rows, cols, rows + cols + n, 0.02)
        mats = [P.Matrix(ty, rows, cols, raw) for _ in range(2)]
        print(f"GEMM {tag}", file=sys.stderr, flush=True)
        x = rng.standard_normal((n, cols)).astype(np.float32)
        q, sa, sums = P.quantize_acts(x)
        dq, ds, dm = P.DeviceArray.from_host(q), P.DeviceArray.from_host(sa), P.DeviceArray.from_host(sums)
        out = P.DeviceArray((n, rows), np.float32)
        for phase, calls in (("warmup", WARMUP), ("timed", TIMED)):
            _marker(P, marker)
            for i in range(calls):
                P.check(P.load().prana_matmul_prefill(mats[i % 2].h, None, dq.ptr, ds.ptr, dm.ptr, n, out.ptr, None))
        _marker(P, marker)
        P.check(P.load().prana_synchronize())
        cases.append({"config": "GEMM", "case": f"{tag} {rows}x{cols} N={n}", "calls": TIMED,
                      "bytes": len(raw) + n * cols + n * rows * 4, "ops": 2 * rows * cols * n})
        del mats

    for tag, rows, cols in (VERIFY_SHAPES if only == "VERIFY" else []):
        # C4's speculative verify batches: Q4_0 7B shapes at k+1 tokens (and
        # 2, 16), pre-quantized activations, weight copies past the MALL
        raw = P.synth_tensor(Q4_0, rows, cols, rows * 3 + cols, 0.02)
        copies = max(3, -(-2 * MALL // raw.nbytes))
        mats = [P.Matrix(Q4_0, rows, cols, raw) for _ in range(copies)]
        print(f"VERIFY {tag}: {copies} copies", file=sys.stderr, flush=True)
        for n in VERIFY_TOKENS:
            q, sa, sums = P.quantize_acts(rng.standard_normal((n, cols)).astype(np.float32))
            dq, ds, dm = P.DeviceArray.from_host(q), P.DeviceArray.from_host(sa), P.DeviceArray.from_host(sums)
            out = P.DeviceArray((n, rows), np.float32)
            for phase, calls in (("warmup", WARMUP), ("timed", TIMED)):
                _marker(P, marker)
                for i in range(calls):
                    P.check(P.load().prana_matmul_prefill(mats[i % copies].h, None, dq.ptr, ds.ptr, dm.ptr, n,
                                                          out.ptr, None))
            _marker(P, marker)
            P.check(P.load().prana_synchronize())
            cases.append({"config": "C4 verify", "case": f"{tag} Q4_0 {rows}x{cols} N={n}", "calls": TIMED,
                          "bytes": len(raw) + n * cols + n * rows * 4})
        del mats

    nh, nkv, hd = 32, 8, 128
    kv = nkv * hd
    lib = P.load()
    for rows in (ATTN_ROWS if only == "ATTN" else []):
        # the 7B decode's attention (32/8 heads, hd 128, f16 cache) on the
        # exact one-launch kernel, one query row at position rows - 1
        print(f"ATTN rows={rows}", file=sys.stderr, flush=True)
        qa = P.DeviceArray.from_host(rng.standard_normal(nh * hd).astype(np.float32))
        ka = P.DeviceArray.from_host(rng.standard_normal((rows, kv)).astype(np.float16).view(np.uint16))
        va = P.DeviceArray.from_host(rng.standard_normal((rows, kv)).astype(np.float16).view(np.uint16))
        oa = P.DeviceArray((nh * hd,), np.float32)
        for phase, calls in (("warmup", WARMUP), ("timed", TIMED)):
            _marker(P, marker)
            for i in range(calls):
                P.check(lib.prana_attention_decode(qa.ptr, ka.ptr, va.ptr, rows - 1, nh, nkv, hd, oa.ptr, None))
        _marker(P, marker)
        P.check(lib.prana_synchronize())
        cases.append({"config": "C4 attention", "case": f"decode over {rows} cache rows, exact", "calls": TIMED,
                      "bytes": 2 * rows * kv * 2 + nh * hd * 8})
    for ctx in (C3_CTX if only in (None, "C3") else []):
        print(f"C3 ctx={ctx}", file=sys.stderr, flush=True)
        rows = ctx + 1
        per_seq = 2 * rows * kv * 2
        # q and the new k row get NeoX RoPE (theta 1e4) at position ctx
        q8 = np.stack([P.rope(r[None, :], ctx, hd, 1e4, True)[0]
                       for r in rng.standard_normal((8, nh * hd)).astype(np.float32)])
        knew = np.stack([P.rope(r[None, :], ctx, hd, 1e4, True)[0]
                         for r in rng.standard_normal((8, kv)).astype(np.float32)])
        kh = rng.standard_normal((rows, kv)).astype(np.float16).view(np.uint16)
        vh = rng.standard_normal((rows, kv)).astype(np.float16).view(np.uint16)
        # cache copies (same values, distinct addresses) rotate past 2 x MALL
        n_cache = max(8, -(-2 * MALL // per_seq))
        kcs, vcs = [], []
        for i in range(n_cache):
            kh[ctx] = P.f32_to_f16(knew[i % 8])
            kcs.append(P.DeviceArray.from_host(kh))
            vcs.append(P.DeviceArray.from_host(vh))
        q = P.DeviceArray.from_host(q8)
        out = P.DeviceArray((8, nh * hd), np.float32)
        pos8 = (C.c_size_t * 8)(*([ctx] * 8))

        def ptrs(lst, i0, n):
            return (C.c_void_p * n)(*[lst[(i0 + j) % n_cache].ptr.value for j in range(n)])

        def exact_b1(i):
            P.check(lib.prana_attention_decode(q.ptr, kcs[i % n_cache].ptr, vcs[i % n_cache].ptr, ctx, nh, nkv, hd,
                                               out.ptr, None))

        def split_b1(i):
            P.check(lib.prana_attention_decode_splitk(q.ptr, ptrs(kcs, i, 1), ptrs(vcs, i, 1), pos8, 1, nh, nkv,
                                                      hd, out.ptr, None))

        def exact_b8(i):
            for j in range(8):
                c = (8 * i + j) % n_cache
                P.check(lib.prana_attention_decode(C.c_void_p(q.ptr.value + j * nh * hd * 4), kcs[c].ptr,
                                                   vcs[c].ptr, ctx, nh, nkv, hd,
                                                   C.c_void_p(out.ptr.value + j * nh * hd * 4), None))

        def split_b8(i):
            P.check(lib.prana_attention_decode_splitk(q.ptr, ptrs(kcs, 8 * i, 8), ptrs(vcs, 8 * i, 8), pos8, 8, nh,
                                                      nkv, hd, out.ptr, None))

        def verify8(i):
            # eight query rows at ctx-7..ctx over one cache (the verify form)
            c = i % n_cache
            P.check(lib.prana_attention_verify(q.ptr, kcs[c].ptr, vcs[c].ptr, ctx - 7, 8, nh, nkv, hd, out.ptr,
                                               None))

        for tag, fn, b in (("decode, exact", exact_b1, 1), ("decode, split-K", split_b1, 1),
                           ("8 query rows at ctx-7..ctx over one cache (verify form), exact", verify8, 1),
                           ("batch 8 (eight independent caches), exact", exact_b8, 8),
                           ("batch 8 (eight independent caches), split-K", split_b8, 8)):
            for phase, calls in (("warmup", WARMUP), ("timed", TIMED)):
                _marker(P, marker)
                for i in range(calls):
                    fn(i)
            _marker(P, marker)
            P.check(lib.prana_synchronize())
            cases.append({"config": "C3", "case": f"ctx={ctx} {tag}", "calls": TIMED,
                          "bytes": b * per_seq + b * nh * hd * 8})
        for a in kcs + vcs:
            a.free()
    with open(manifest_path, "w") as f:
        json.dump(cases, f, indent=1)
    print(f"wrote {len(cases)} cases to {manifest_path}", file=sys.stderr)


def run_models():
    """End-to-end passes of the model configurations (wall clock of the
    library's own prefill / decode timers; weights random-init, synthetic
    prompts): C0 greedy decode, C2 2048-token prefill + 512-token decode, C4
    plain and speculative (k = 4, 8) decode after a 512-token prefill."""
    import prana_amd as P
    from prana_amd import models as M

    rng = np.random.default_rng(20261202)
    rows = []

    def rec(config, case, st, extra=None):
        r = {"config": config, "case": case, "prompt_tokens": st.prompt_tokens,
             "generated_tokens": st.generated_tokens,
             "prefill_tok_s": round((st.prompt_tokens - 1) / st.prefill_seconds, 1) if st.prefill_seconds > 0 else None,
             "decode_tok_s": round(st.generated_tokens / st.decode_seconds, 1) if st.decode_seconds > 0 else None}
        r.update(extra or {})
        rows.append(r)
        print(json.dumps(r), file=sys.stderr, flush=True)

    g = P.Model(M.C0, M.c0_tensors(seed=1))
    prompt = rng.integers(0, M.C0["vocab_size"], 5).astype(np.uint32)
    g.generate(prompt, 16)
    _, st = g.generate(prompt, 256)
    rec("C0", "15M shape, Q8_0, 5-token prompt, greedy to position 256", st)
    del g

    g = P.Model(M.C2, M.c2_tensors(seed=2))
    prompt = rng.integers(0, M.C2["vocab_size"], 2048).astype(np.uint32)
    g.generate(prompt[:64], 8)
    _, st = g.generate(prompt, 512)
    rec("C2", "qwen2-0.5B shape, Q4_K/Q6_K mix, 2048-token prefill + 512 greedy tokens", st)
    del g

    g = P.Model(M.C4, M.c4_tensors(seed=4))
    dcfg = M.c4_draft_config()
    draft = P.Model(dcfg, M.synth_tensors(dcfg, M.types_c0, 1))
    prompt = rng.integers(0, M.C4["vocab_size"], 512).astype(np.uint32)
    g.generate(prompt[:16], 4)
    plain, st = g.generate(prompt, 128)
    rec("C4", "7B shape, Q4_0, 512-token prefill + 128 greedy tokens", st)
    for k in (4, 8):
        spec, st = P.generate_speculative(g, draft, prompt, 128, k)
        rec("C4", f"speculative, 15M-shape draft, k={k}", st,
            {"proposed": st.proposed, "accepted": st.accepted, "equals_plain": bool(list(spec) == list(plain))})
    return rows


def run_spec(k, tokens):
    """C4 speculative decode alone (for a kernel trace of its rounds): the C4
    target and draft of run_models, a 512-token prefill, a warm-up call, then
    one timed call of `tokens` tokens with k drafts per round."""
    import prana_amd as P
    from prana_amd import models as M

    g = P.Model(M.C4, M.c4_tensors(seed=4))
    dcfg = M.c4_draft_config()
    draft = P.Model(dcfg, M.synth_tensors(dcfg, M.types_c0, 1))
    prompt = np.random.default_rng(20261202).integers(0, M.C4["vocab_size"], 512).astype(np.uint32)
    P.generate_speculative(g, draft, prompt[:64], 8, k)
    _, st = P.generate_speculative(g, draft, prompt, tokens, k)
    print(json.dumps({"config": "C4", "k": k, "generated_tokens": st.generated_tokens, "proposed": st.proposed,
                      "accepted": st.accepted,
                      "decode_tok_s": round(st.generated_tokens / st.decode_seconds, 1)}), flush=True)


def run_c2_decode(tokens):
    """C2 decode alone (for a kernel trace of its steps): the qwen2-0.5B-shape
    model of run_models, a warm-up call, then one timed generate call with a
    2048-token prompt (2047-token prefill) and `tokens` greedy tokens."""
    import prana_amd as P
    from prana_amd import models as M

    g = P.Model(M.C2, M.c2_tensors(seed=2))
    prompt = np.random.default_rng(20261202).integers(0, M.C2["vocab_size"], 2048).astype(np.uint32)
    g.generate(prompt[:64], 8)
    _, st = g.generate(prompt, tokens)
    print(json.dumps({"config": "C2", "generated_tokens": st.generated_tokens,
                      "decode_tok_s": round(st.generated_tokens / st.decode_seconds, 1)}), flush=True)


def models_table(rows):
    out = ["| config | case | prefill tok/s | decode tok/s | note |", "|---|---|---:|---:|---|"]
    for r in rows:
        note = ""
        if "proposed" in r:
            note = f"accepted {r['accepted']}/{r['proposed']} drafts; stream equals plain greedy: {r['equals_plain']}"
        out.append(f"| {r['config']} | {r['case']} | {r['prefill_tok_s']} | {r['decode_tok_s']} | {note} |")
    return "\n".join(out)


def summarize(db, manifest_path):
    cases = json.load(open(manifest_path))
    c = sqlite3.connect(db)
    rows = c.execute("select name, duration from kernels order by start").fetchall()
    segs, cur = [], None
    for name, dur in rows:
        if "fillBuffer" in name:
            if cur is not None:
                segs.append(cur)
            cur = []
        elif cur is not None:
            cur.append((name, dur))
    if cur is not None:
        segs.append(cur)
    # three segments per case: warmup, timed, then set-up of the next case
    out = ["| config | case | kernels per call | us per call | GB/s | % of 8 TB/s | int8 TOPS | % of 5 POPS |",
           "|---|---|---|---:|---:|---:|---:|---:|"]
    for i, cs in enumerate(cases):
        seg = segs[3 * i + 1]
        work = [(n, d) for n, d in seg if "__amd_rocclr" not in n]
        names = sorted({n.replace("void ", "").replace("(anonymous namespace)::", "").replace("prana::", "").split("(")[0]
                        for n, _ in work})
        us = sum(d for _, d in work) / 1000.0 / cs["calls"]
        gbs = cs["bytes"] / (us * 1e-6) / 1e9
        tops = cs["ops"] / (us * 1e-6) / 1e12 if "ops" in cs else None
        ops_cols = f"| {tops:.1f} | {100 * tops / 5000:.1f}% |" if tops else "| | |"
        out.append(f"| {cs['config']} | {cs['case']} | {', '.join('`' + n + '`' for n in names)} | {us:.2f} | {gbs:.0f} "
                   f"| {100 * gbs / 8000:.1f}% {ops_cols}")
    print("\n".join(out))


def summarize_counters(db, cus=256, xcds=8):
    """Per-kernel MFMA / VALU utilisation from a rocprofv3 --pmc run with
    SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_I8
    SQ_ACTIVE_INST_VALU SQ_BUSY_CYCLES. rocprofv3 reports GRBM_GUI_ACTIVE
    summed over the XCDs, so a dispatch's active cycles are that sum / xcds
    (the implied clock, cycles over the dispatch's duration, is printed as a
    check). MfmaUtil: busy cycles over active cycles x SIMDs; VALU busy per
    SIMD: each VALU instruction (SQ_ACTIVE_INST_VALU counts one per
    instruction) holds its SIMD four cycles; int8 MFMA ops = MOPS x 512."""
    import collections
    import re
    c = sqlite3.connect(db)
    rows = c.execute("select dispatch_id, kernel_name, grid_size, counter_name, value, duration "
                     "from counters_collection").fetchall()
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    names, durs = {}, {}
    for did, kn, gs, cn, v, dur in rows:
        per[did][cn] = max(per[did][cn], v) if cn == "GRBM_GUI_ACTIVE" else per[did][cn] + v
        kk = kn.replace("(anonymous namespace)::", "").replace("prana::", "")
        names[did] = (re.sub(r"^void ", "", kk.split("(")[0]), gs)
        durs[did] = dur
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    for did, d in per.items():
        for cn, v in d.items():
            agg[names[did]][cn].append(v)
        agg[names[did]]["_dur_ns"].append(durs[did])
    out = ["| kernel | grid | dispatches | us | implied clock GHz | MfmaUtil % | VALU busy % per SIMD "
           "| int8 MFMA ops / dispatch |", "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for (k, gs), d in sorted(agg.items()):
        if "gemm" not in k and "gemv" not in k:
            continue
        n = len(d["GRBM_GUI_ACTIVE"])
        cyc = sum(d["GRBM_GUI_ACTIVE"]) / n / xcds
        dur = sum(d["_dur_ns"]) / n
        mfma = sum(d["SQ_VALU_MFMA_BUSY_CYCLES"]) / n
        valu = sum(d["SQ_ACTIVE_INST_VALU"]) / n
        mops = sum(d["SQ_INSTS_VALU_MFMA_MOPS_I8"]) / n * 512
        out.append(f"| `{k}` | {int(gs)} | {n} | {dur / 1e3:.1f} | {cyc / dur:.2f} | "
                   f"{100 * mfma / (cyc * 4 * cus):.1f} | {100 * valu / cus / cyc:.1f} | {mops:.3e} |")
    print("\n".join(out))


def attention_counters(dbs, cus=256):
    """Per attention kernel (grid) from rocprofv3 --pmc runs of --only ATTN:
    texture-address (TA) busy cycles per active compute unit (one workgroup
    per CU) next to the kernel's GRBM active cycles per XCD, VALU and LDS
    instructions per wave, and LDS bank-conflict and active cycles per CU."""
    import collections
    import re
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    names = {}
    for db in dbs:
        c = sqlite3.connect(db)
        for did, kn, gs, wg, cn, v in c.execute(
                "select dispatch_id, kernel_name, grid_size, workgroup_size, counter_name, value from counters_collection"):
            key = (db, did)
            per[key][cn] = max(per[key][cn], v) if cn == "GRBM_GUI_ACTIVE" else per[key][cn] + v
            kk = kn.replace("(anonymous namespace)::", "").replace("prana::", "")
            names[key] = (re.sub(r"^void ", "", kk.split("(")[0]), int(gs), int(wg))
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    for key, d in per.items():
        for cn, v in d.items():
            agg[names[key]][cn].append(v)
    med = lambda v: sorted(v)[len(v) // 2] if v else float("nan")
    out = ["| kernel | grid | workgroups | GRBM active cycles | TA busy cycles / CU | VALU insts / wave | LDS insts / wave "
           "| LDS bank-conflict cycles / CU | LDS active cycles / CU |", "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for (k, gs, wg), d in sorted(agg.items()):
        if "attn" not in k:
            continue
        wgs = gs // wg
        waves = med(d.get("SQ_WAVES", [])) or 1
        act = min(wgs, cus)
        out.append(f"| `{k}` | {gs} | {wgs} | {med(d.get('GRBM_GUI_ACTIVE', [])):.0f} | "
                   f"{med(d.get('TA_TA_BUSY_sum', [])) / act:.0f} | {med(d.get('SQ_INSTS_VALU', [])) / waves:.0f} | "
                   f"{med(d.get('SQ_INSTS_LDS', [])) / waves:.0f} | {med(d.get('SQ_LDS_BANK_CONFLICT', [])) / act:.0f} | "
                   f"{med(d.get('SQ_LDS_IDX_ACTIVE', [])) / act:.0f} |")
    print("\n".join(out))


def decode_trace_summary(db, bench_json, command):
    """Markdown summary of a kernel trace of bench.py (7B-shape Q4_0 decode):
    per-kernel time over the run, the decode GEMVs by shape (grid size), and
    the bench's own event-sampled GEMV figures from its JSON line."""
    import re
    from collections import defaultdict

    c = sqlite3.connect(db)
    rows = c.execute("select name, count(*), avg(duration), min(duration), max(duration), sum(duration) from kernels "
                     "group by name order by sum(duration) desc").fetchall()
    tot = sum(r[5] for r in rows)

    def short(n):
        n = n.replace("prana::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")
        return re.sub(r"\(.*$", "", n.replace("prana::", "").replace("void ", ""))

    out = ["# 7B-shape Q4_0 decode: rocprofv3 kernel trace", "",
           "Command (from the repository root on the GPU box; `$REPO` is that root):", "", "```", command, "```", "",
           "Kernel time per kernel over the whole run (model upload, 511-token prefill, warmup and timed decode steps).",
           "", "| kernel | calls | avg us | min us | max us | total ms | share |", "|---|---:|---:|---:|---:|---:|---:|"]
    for n, cnt, avg, mn, mx, sm in rows[:16]:
        out.append(f"| `{short(n)}` | {cnt} | {avg / 1000:.2f} | {mn / 1000:.2f} | {mx / 1000:.2f} | {sm / 1e6:.2f} "
                   f"| {100 * sm / tot:.1f}% |")
    out.append(f"| (all kernels) | {sum(r[1] for r in rows)} | | | | {tot / 1e6:.2f} | 100% |")
    shapes = {("gemv_tile_kernel<3, 4, false, false, 1024, true, false>", 192 * 1024):
              ("rmsnorm + Q\\|K\\|V 6144x4096 + RoPE", 14.16),
              ("gemv_tile_kernel<3, 4, false, false, 256, false, false>", 512 * 256): ("wo 4096x4096", 9.44),
              ("gemv_tile_kernel<3, 4, true, true, 1024, true, true>", 225 * 1024):
              ("rmsnorm + gate\\|up 2x14336x4096 + SiLU + quantize", 66.06),
              ("gemv_tile_kernel<3, 7, false, false, 256, false, false>", 1024 * 256): ("down 4096x14336", 33.03),
              ("gemv_tile_kernel<3, 4, false, false, 256, false, false>", 4000 * 256): ("LM head 32000x4096", 73.73)}
    d = defaultdict(list)
    for name, dur, gx in c.execute("select name, duration, grid_x from kernels where name like '%gemv_tile_kernel%'"):
        d[(short(name), gx)].append(dur / 1000)
    out += ["", "Decode GEMVs by shape (the grid size identifies the shape; MB = GGUF Q4_0 block bytes streamed):", "",
            "| kernel instance | shape | launches | avg us | MB | GB/s | % of 8 TB/s |", "|---|---|---:|---:|---:|---:|---:|"]
    tok_us = tok_mb = 0.0
    for key, (label, mb) in shapes.items():
        v = d.get(key)
        if not v:
            continue
        a = sum(v) / len(v)
        gbs = mb * 1e3 / a
        mult = 1 if "head" in label else 32
        tok_us += a * mult
        tok_mb += mb * mult
        out.append(f"| `{key[0]}` | {label} | {len(v)} | {a:.2f} | {mb:.2f} | {gbs:.0f} | {100 * gbs / 8000:.1f}% |")
    if tok_us:
        gbs = tok_mb * 1e3 / tok_us
        out.append(f"| per token (32 layers + head, 129 launches) | | | {tok_us:.1f} | {tok_mb:.1f} | {gbs:.0f} "
                   f"| {100 * gbs / 8000:.1f}% |")
    b = json.loads(open(bench_json).read().strip().splitlines()[-1])
    r = b["roofline"]
    out += ["", "The bench itself (no profiler attached) samples every 8th GEMV dispatch with HIP dispatch-timestamp "
            f"events inside its timed region ({b['value']} tok/s, {b['config']['tok_s_without_events']} tok/s with no "
            "events):", "", "| projection | launches | avg us | GB/s | % of 8 TB/s | us per token |",
            "|---|---:|---:|---:|---:|---:|"]
    for p in r.get("per_projection", []):
        out.append(f"| {p['name'].replace('|', chr(92) + '|')} | {p['launches']} | {p['avg_us']} | {p['gbs']} "
                   f"| {100 * p['frac']:.1f}% | {p['us_per_token']} |")
    out += ["", f"The roofline object names the projection with the most time per token: {r['kernel']}, "
            f"{r['avg_launch_us']} us, {r['achieved']} GB/s ({100 * r['frac']:.1f} % of 8 TB/s)."]
    if r.get("traffic"):
        out[-1] += (f" Its HBM traffic per launch from the counter runs is "
                    f"{r['traffic'] / r['bytes_per_launch']:.3f} x the algorithmic bytes "
                    f"(q4_0_gemv_7b_decode_traffic.json).")
    print("\n".join(out))


def traffic_summary(fetch_db, write_db, commands):
    """HBM bytes per decode-GEMV launch of the 7B-shape bench, by projection,
    from two rocprofv3 --pmc runs of `bench.py --copy-calibration` (FETCH_SIZE,
    then WRITE_SIZE; KiB per dispatch), each scaled by what the same counter
    reads for the bench's 512 MiB device-to-device calibration copy. Prints the
    JSON that bench.py reads for its roofline's `traffic`."""
    from collections import defaultdict

    def load(f):
        return sqlite3.connect(f).execute(
            "select dispatch_id, kernel_name, grid_size, value from counters_collection").fetchall()

    F, Wr = load(fetch_db), load(write_db)
    nb = 512 << 20
    ffac = max(v for _, n, _, v in F if "copyBuffer" in n) * 1024 / nb
    wfac = max(v for _, n, _, v in Wr if "copyBuffer" in n) * 1024 / nb
    q4 = lambda r, c: r * c // 32 * 18
    fam = {("false, false, 1024, true, false>", 192 * 1024): ("Q|K|V + attention rmsnorm", q4(6144, 4096)),
           ("4, false, false, 256, false, false>", 512 * 256): ("wo", q4(4096, 4096)),
           ("true, true, 1024, true, true>", 225 * 1024): ("gate|up + SiLU + FFN rmsnorm", 2 * q4(14336, 4096)),
           ("7, false, false, 256, false, false>", 1024 * 256): ("down", q4(4096, 14336)),
           ("4, false, false, 256, false, false>", 4000 * 256): ("LM head", q4(32000, 4096))}

    def classify(name, gs):
        if "gemv_tile_kernel<3" not in name:
            return None
        for (sig, g), v in fam.items():
            if sig in name and gs == g:
                return v
        return None

    agg = defaultdict(lambda: [0, 0.0, 0.0])
    for rows, idx, fac in ((F, 1, ffac), (Wr, 2, wfac)):
        for _, name, gs, v in rows:
            c = classify(name, gs)
            if c is None:
                continue
            a = agg[c[0]]
            if idx == 1:
                a[0] += 1
            a[idx] += v * 1024 / fac
    out = {"workload": "7B-shape Q4_0 decode (bench.py): the decode weight GEMV launches (gemv_tile_kernel "
                       "instances), split by projection; the Q|K|V and gate|up launches also compute their input's "
                       "rmsnorm (the gate|up launch in its leading norm workgroup)",
           "hbm_bytes_per_launch": {}, "per_projection": {}}
    for _, (label, alg) in fam.items():
        a = agg.get(label)
        if not a or a[0] == 0:
            continue
        fetch, write = a[1] / a[0], a[2] / a[0]
        out["hbm_bytes_per_launch"][label] = round(fetch + write)
        out["per_projection"][label] = {"dispatches": a[0], "algorithmic_bytes": alg, "fetch_bytes": round(fetch),
                                        "write_bytes": round(write), "fetch_vs_algorithmic": round(fetch / alg, 4)}
    out["scaling"] = {"method": "FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled by what the same counters read "
                                "for a 512 MiB device-to-device copy (bench.py --copy-calibration, kernel "
                                "__amd_rocclr_copyBuffer)",
                      "fetch_counter_per_true_byte": round(ffac, 4), "write_counter_per_true_byte": round(wfac, 4)}
    out["commands"] = commands
    print(json.dumps(out, indent=1))


def round_trace_summary(db):
    """Per-kernel table of the last timed call in a kernel trace of --spec:
    every kernel after the call's prefill (the last prefill-GEMM or prefill
    attention launch), grouped by kernel, grid and LDS size."""
    from collections import defaultdict

    c = sqlite3.connect(db)
    rows = c.execute("select name, start, end, grid_x, workgroup_x, lds_size from kernels order by start").fetchall()
    last = max(i for i, r in enumerate(rows) if "attn_prefill" in r[0] or "gemm_mfma" in r[0])
    tail = rows[last + 1:]
    d = defaultdict(lambda: [0, 0.0])
    for n, st, en, gx, wx, lds in tail:
        n = n.replace("(anonymous namespace)::", "").replace("void ", "").replace("prana::", "")
        key = (n.split("(")[0], gx // wx, wx, lds)
        d[key][0] += 1
        d[key][1] += (en - st) / 1000
    tot = sum(v[1] for v in d.values())
    out = [f"Kernel time {tot / 1000:.1f} ms over a {(tail[-1][2] - tail[0][1]) / 1e6:.1f} ms span, "
           f"{len(tail)} launches.", "",
           "| kernel | grid | lanes | LDS bytes | launches | avg us | total ms | share |",
           "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for k, v in sorted(d.items(), key=lambda kv: -kv[1][1])[:18]:
        out.append(f"| `{k[0]}` | {k[1]} | {k[2]} | {k[3]} | {v[0]} | {v[1] / v[0]:.2f} | {v[1] / 1000:.2f} "
                   f"| {100 * v[1] / tot:.1f}% |")
    print("\n".join(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--summarize", metavar="DB")
    ap.add_argument("--counters", metavar="DB", help="MFMA / VALU utilisation table of a --pmc run")
    ap.add_argument("--models", action="store_true", help="end-to-end C0 / C2 / C4 passes instead of the kernel sweep")
    ap.add_argument("--only", choices=["C1", "GEMM", "C3", "VERIFY", "ATTN"], help="run one configuration's sweep")
    ap.add_argument("--attn-counters", nargs="+", metavar="DB", help="attention counter table of --pmc runs of --only ATTN")
    ap.add_argument("--spec", type=int, metavar="K", help="C4 speculative decode alone, K drafts per round")
    ap.add_argument("--tokens", type=int, default=48, help="tokens of the --spec or --c2-decode call")
    ap.add_argument("--c2-decode", action="store_true", help="C2 decode alone (2048-token prompt, --tokens steps)")
    ap.add_argument("--round-trace", metavar="DB", help="per-kernel table of a kernel trace of --spec or --c2-decode")
    ap.add_argument("--decode-trace", nargs=3, metavar=("DB", "BENCH_JSON", "COMMAND"),
                    help="summary of a kernel trace of bench.py (with the bench's JSON line and the trace command)")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                    help="HBM traffic JSON of two --pmc runs (FETCH_SIZE, WRITE_SIZE) of bench.py --copy-calibration")
    ap.add_argument("--traffic-commands", nargs="*", default=[], help="the commands recorded in the --traffic JSON")
    ap.add_argument("--manifest", default=os.path.join(os.getcwd(), "microbench_cases.json"))
    args = ap.parse_args()
    if args.models:
        print(models_table(run_models()))
    elif args.spec:
        run_spec(args.spec, args.tokens)
    elif args.c2_decode:
        run_c2_decode(args.tokens)
    elif args.round_trace:
        round_trace_summary(args.round_trace)
    elif args.decode_trace:
        decode_trace_summary(*args.decode_trace)
    elif args.traffic:
        traffic_summary(*args.traffic, args.traffic_commands)
    elif args.counters:
        summarize_counters(args.counters)
    elif args.attn_counters:
        attention_counters(args.attn_counters)
    elif args.summarize:
        summarize(args.summarize, args.manifest)
    else:
        run(args.manifest, args.only)


if __name__ == "__main__":
    main()

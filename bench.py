"""Decode throughput of the MI355X decode loop on the Llama-3-8B shape.

Workload (default): Llama-3.1-8B-shaped decoder (32 layers, d_model 4096,
32 query / 8 KV heads of 128, SwiGLU 14336, vocab 128256, RoPE theta 5e5),
int4 group-32 weights generated on the device from a seed, a 4096-token
fp16 paged KV context (16-token pages, shuffled block table) of N(0,1)
values, greedy decode at batch 1.  One step = one decode_step (every
layer, lm_head and argmax) of every sequence, as one HIP graph launch;
W untimed warmup steps, then K timed steps, bracketed by device syncs.

Also reported:
  roofline      the dominant kernel (fused RMSNorm + gate/up int4 GEMV +
                SwiGLU of one layer) timed with HIP events over back-to-back
                launches on the library stream; achieved = its algorithmic
                bytes / average duration, against 8 TB/s HBM peak.
  attention     the fp16 paged attention kernel of one layer, same method.
  cpu_baseline  the C oracle (OpenMP) on the host cores, on a bounded
                sample: one 8B-shaped layer at 4096 context plus 1/8 of the
                lm_head rows, scaled to a token (32 layers + full lm_head).
  nxf_verify    XXH32 verification of NXF chunks on the GPU (k_xxh32): 4 GiB
                (an 8B model's weight bytes) as 64 KiB chunks, HIP-event
                timed, against the oracle's XXH32 on one host core.
  prefill       batched prefill of a 2048-token prompt on a fresh model of
                the same shape (dense models), wall clock around the call;
                its dominant kernel, the gate/up int4-g32 GEMM of a
                2048-token chunk, against the 2.5 PFLOP/s dense fp16 peak.
  sampling      decode steps with temperature / top-k / top-p sampling
                inside the step graph, and the oracle sampler's time.
  tiering       one layer of the same shape at a 32768-token context with
                fp16, TurboQuant and tiered pages (last 4096 positions
                fp16): attention time and KV bytes, one-layer step time.

Other workloads: --model mixtral-8x7b (top-2 of 8 experts of 14336, vocab
32000; the roofline kernel is then the routed gate/up expert GEMV), --kv tq
(TurboQuant pages), --kv tiered [--hot-window H], --batch, --ctx.
--decode-only leaves out the GEMV, NXF, prefill and tiering lines.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B]
                       [--model llama-8b|mixtral-8x7b] [--kv fp16|tq|tiered --ctx C]
                       [--hot-window H] [--no-cpu] [--decode-only]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "nexus-inference-engine-_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "decode tok/s, Llama-3-8B-shape int4 bs1 ctx4K; GEMV/attn HBM GB/s % of peak"
PEAK_HBM_GBS = 8000.0

LLAMA8B = dict(n_layers=32, d_model=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336,
               vocab=128256, n_experts=0, top_k=0, batch=1, kv_kind=0, rope_theta=500000.0,
               eps=1e-5, seed=0x5EED)
# Mixtral-8x7B shape: 8 SwiGLU experts of 14336, router top-2, vocab 32000
MIXTRAL = dict(LLAMA8B, vocab=32000, n_experts=8, top_k=2, rope_theta=1000000.0)
MODELS = {"llama-8b": LLAMA8B, "mixtral-8x7b": MIXTRAL}


def cpu_baseline(base: dict, ctx_len: int, batch: int, kv_kind: int, hot_window: int = 0, reps: int = 3,
                 plans=None) -> dict:
    """Time the oracle's decode step on a bounded sample and scale to a step:
    decode steps of one layer of the shape plus 1/8 of the lm_head rows,
    scaled to every layer and the whole lm_head.  plans: list of (threads,
    steps, seconds) -- at `threads` OpenMP threads (0: all), `steps` decode
    steps, fewer once `seconds` of sampled work have passed (0: no limit);
    the model is built once and the result is one baseline per plan (a
    single one at the current thread count and `reps` steps by default)."""
    import numpy as np

    import oracle
    single = plans is None
    plans = plans or [(0, reps, 0.0)]
    vocab_frac = 8
    cfg = dict(base, n_layers=1, vocab=base["vocab"] // vocab_frac, batch=batch, kv_kind=kv_kind,
               max_seq=((ctx_len + sum(p[1] + 1 for p in plans) + 16) // 16 + 1) * 16, hot_window=hot_window)
    m = oracle.Model(**cfg)
    m.fill_context(ctx_len, 4 if kv_kind else 0)
    tok = np.zeros(batch, np.int32)
    shape = "8B-shaped" if base["n_experts"] == 0 else "Mixtral-shaped (top-2 of 8 experts)"
    kv = ["fp16", "TurboQuant", "tiered"][kv_kind]

    def run(steps, budget):
        m.forward_timed(tok)  # warm caches
        tl, th, n = 0.0, 0.0, 0
        while n < steps:
            _, a, b = m.forward_timed(tok)
            tl += a
            th += b
            n += 1
            if budget and tl + th > budget:
                break
        t_step = base["n_layers"] * tl / n + vocab_frac * th / n
        return {"value": round(batch / t_step, 4), "unit": "tok/s",
                "cores": int(oracle.lib.nxo_num_threads()), "kind": "port",
                "sample": (f"{n} oracle decode steps of one {shape} layer at batch {batch}, ctx {ctx_len} {kv} "
                           f"pages + lm_head rows 1/{vocab_frac}, scaled to {base['n_layers']} layers + full lm_head")}
    try:
        out = [with_threads(t, lambda: run(st, bud)) for t, st, bud in plans]
    finally:
        m.close()
    return out[0] if single else out


TINY = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=688, vocab=4096,
            n_experts=0, top_k=0, batch=1, kv_kind=0, rope_theta=10000.0, eps=1e-5, seed=0x5EED)


def seeded_prompt(seed: int, batch: int, P: int, vocab: int):
    """Uniform token ids in [4, vocab) from a seeded generator."""
    import numpy as np
    return np.random.default_rng(seed).integers(4, vocab, (batch, P), dtype=np.int32)


def cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def with_threads(n: int, fn):
    """fn() with the oracle's OpenMP pool at n threads (0: all), restored after."""
    import oracle
    before = int(oracle.lib.nxo_num_threads())
    if n > 0:
        oracle.lib.nxo_set_num_threads(n)
    try:
        return fn()
    finally:
        oracle.lib.nxo_set_num_threads(before)


def cpu_baselines(base: dict, ctx_len: int, batch: int, kv_kind: int, hot_window: int) -> dict:
    """The oracle on the host at all cores and at one core: the main
    workload (bounded sample, scaled to a token), the tiny model's full
    greedy decode (config 1) and the five GEMV shapes at batch 1 and 8
    (config 2, one product each)."""
    import numpy as np

    import oracle
    allc = int(oracle.lib.nxo_num_threads())
    out = {"cpu_model": cpu_model_name(), "cores_all": allc}
    out["decode_1core"] = with_threads(1, lambda: cpu_baseline(base, ctx_len, batch, kv_kind, hot_window, reps=1))

    def tiny():
        m = oracle.Model(**dict(TINY, max_seq=128))
        prompt = seeded_prompt(TINY["seed"], 1, 16, TINY["vocab"])
        t0 = time.perf_counter()
        m.generate(prompt, 64)
        dt = time.perf_counter() - t0
        m.close()
        return round(64 / dt, 2)
    out["tiny_decode"] = {"workload": "tiny Llama (2 layers, d 256), 16-token prompt + 64 greedy tokens",
                          "unit": "tok/s", "all_cores": with_threads(0, tiny), "one_core": with_threads(1, tiny)}
    rng = np.random.default_rng(0)
    gem = []
    for N, K in GEMV_SHAPES:
        G = (K + 31) // 32
        codes = rng.integers(0, 256, (N, G * 16), dtype=np.uint8)
        scales = np.full((N, G), 0x2000, np.uint16)  # fp16 2^-7
        row = {"shape": f"{N}x{K}"}
        for B in (1, 8):
            x = rng.standard_normal((B, K)).astype(np.float32)
            nbytes = N * K * 0.5625 + B * (2 * K + 2 * N)
            for tag, n in (("all", 0), ("1core", 1)):
                def one():
                    t0 = time.perf_counter()
                    oracle.gemv(codes, scales, x, N, K)
                    return time.perf_counter() - t0
                dt = with_threads(n, one)
                row[f"b{B}_{tag}_us"] = round(dt * 1e6, 1)
                row[f"b{B}_{tag}_GBps"] = round(nbytes / dt / 1e9, 2)
        gem.append(row)
    out["gemv"] = gem
    return out


def decode_line(ctx, base: dict, name: str, batch: int, kv_kind: int, ctx_len: int, steps: int,
                prompt: bool = False, cpu: bool = False) -> dict:
    """Greedy decode rate of one more workload: its model built on the
    device, its context filled with seeded K/V (or, with `prompt`, a seeded
    prompt of ctx_len tokens prefilled), 2 untimed steps, then `steps` timed
    (device synchronized on both sides); bytes per step are the algorithmic
    weight and KV bytes.  cpu: the oracle's rate on the same workload (8
    sampled decode steps at all host cores, up to 8 within 10 s at one core;
    cpu_baseline) and its effective GB/s by the same byte count."""
    import nexus_amd
    max_seq = ((ctx_len + steps + 32) // 16 + 1) * 16
    m = nexus_amd.Model(ctx, **dict(base, batch=batch, kv_kind=kv_kind, max_seq=max_seq))
    if prompt:
        m.prefill(seeded_prompt(base["seed"], batch, ctx_len, base["vocab"]))
    else:
        m.fill_context(ctx_len, 4 if kv_kind else 0)
    m.decode_untimed(2)
    b0 = m.step_bytes()
    ctx.sync()
    t0 = time.perf_counter()
    m.decode_untimed(steps)
    ctx.sync()
    dt = time.perf_counter() - t0
    b1 = m.step_bytes()
    m.close()
    sb = 0.5 * (b0 + b1)
    line = {"workload": name, "batch": batch, "ctx": ctx_len, "steps": steps,
            "tok_s": round(steps * batch / dt, 2), "ms_per_step": round(dt * 1e3 / steps, 4),
            "GB_per_step": round(sb / 1e9, 4), "hbm_GBps_end_to_end": round(sb / (dt / steps) / 1e9, 1),
            "roofline_end_to_end_frac": round(sb / (dt / steps) / 1e9 / PEAK_HBM_GBS, 4)}
    if cpu:
        cbs = cpu_baseline(base, ctx_len, batch, kv_kind, plans=[(0, 8, 0.0), (1, 8, 10.0)])
        for key, cb in zip(("cpu_baseline", "cpu_baseline_1core"), cbs):
            cb["effective_GBps"] = round(sb * cb["value"] / batch / 1e9, 3)
            line[key] = cb
    return line


def measured_traffic(kind: str, nbytes: float):
    """HBM bytes per launch of `kind` ("ffn" / "attention" / "attention_tq")
    from the committed rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE,
    calibrated on a copy kernel); None when no summary is present or it was
    taken on a launch of other algorithmic bytes than `nbytes`."""
    try:
        with open(ROOT / "profiles" / "traffic.json") as f:
            k = json.load(f)["kernels"][kind]
        if abs(k["algorithmic_bytes"] - nbytes) > 1e-3 * nbytes:
            return None
        return int(k["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


GEMV_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]


def gemv_microbench(ctx, batch: int = 1, iters: int = 200) -> list:
    """Standalone int4-g32 GEMV (fp16 x, fp16 y) on the five 8B projection
    shapes; bytes = N*K*0.5625 + batch*(2K + 2N).  The launches are captured
    as one graph and timed with HIP events around its replay, so `us` is a
    launch's share of a graph (what a decode step pays per launch, the
    kernel boundary included).  Each shape rotates over enough weight copies
    (>= 768 MB in total) that every launch reads its weights from HBM, not
    from the 256 MB last-level cache."""
    import ctypes as C
    out = []
    for N, K in GEMV_SHAPES:
        G = (K + 31) // 32
        wbytes = N * G * 18
        ncopies = max(2, -(-(768 << 20) // wbytes))
        ws = [ctx.alloc(N * G * 16) for _ in range(ncopies)]
        ss = [ctx.alloc(N * G * 2) for _ in range(ncopies)]
        x, y = ctx.alloc(batch * K * 2), ctx.alloc(batch * N * 2)
        warr = (C.c_uint64 * ncopies)(*ws)
        sarr = (C.c_uint64 * ncopies)(*ss)
        ms = C.c_double()
        ctx.check(ctx.L.nx_time_gemv(ctx.h, x, warr, sarr, ncopies, y, N, K, batch, iters, C.byref(ms)),
                  "nx_time_gemv")
        nbytes = N * K * 0.5625 + batch * (2 * K + 2 * N)
        gbs = nbytes / (ms.value * 1e-3) / 1e9
        out.append({"shape": f"{N}x{K}", "batch": batch, "us": round(ms.value * 1e3, 3),
                    "GBps": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)})
        for b in ws + ss + [x, y]:
            ctx.free(b)
    return out


def nxf_verify_bench(ctx, cpu: bool, nbytes: int = 4 << 30, chunk: int = 64 << 10, iters: int = 10) -> dict:
    """GB/s of hashing nbytes of device memory as consecutive chunks (the
    load-time verification of an NXF file's chunks); algorithmic bytes =
    the chunk bytes, read once."""
    from nexus_amd.nxf import time_xxh32
    buf = ctx.alloc(nbytes)
    ms, _ = time_xxh32(ctx, buf, nbytes, chunk, iters)
    ctx.free(buf)
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"kernel": "k_xxh32 (XXH32 of NXF chunks, 4 lanes per chunk)", "bytes": nbytes,
           "chunk_bytes": chunk, "avg_us": round(ms * 1e3, 3), "achieved": round(gbs, 1),
           "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}
    if cpu:
        import ctypes as C

        import numpy as np

        import oracle
        sample = np.random.default_rng(0).integers(0, 256, 512 << 20, dtype=np.uint8)
        ptr = sample.ctypes.data
        t0 = time.perf_counter()
        for off in range(0, sample.size, chunk):
            oracle.lib.nxo_xxh32(C.c_void_p(ptr + off), chunk, 0)
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(sample.size / dt / 1e9, 3), "unit": "GB/s", "cores": 1,
                               "kind": "port", "sample": "512 MiB of random bytes as 64 KiB chunks, "
                               "oracle XXH32 (nxo_xxh32) on one host core"}
    return out


PEAK_MFMA_TFLOPS = 2500.0  # dense fp16 matrix-core peak


def tiering_bench(ctx, base: dict, ctx_len: int = 32768, hot_window: int = 4096, steps: int = 64,
                  warm_window: int = 4096, cool_window: int = 8192) -> dict:
    """One layer of the model's shape at a long context, with fp16,
    TurboQuant and tiered pages (two tiers; three: Warm range warm_window;
    evicting: also a Cool window, older pages evicted): the attention pass
    (KV bytes it reads, its time), the time of a one-layer decode step (for
    tiered pages it includes the device compressors, which encode a page
    every 16 steps) and the KV bytes one layer holds for the sequence at the
    end (resident_bytes: pages that hold data, by tier)."""
    import nexus_amd
    out = {"ctx": ctx_len, "hot_window": hot_window, "warm_window": warm_window, "cool_window": cool_window}
    hkv = base["n_kv_heads"]
    per = {"f16": 2 * hkv * base["head_dim"] * 2, "tq": 2 * hkv * 58, "cool": 2 * hkv * 50}
    for name, kind, W, C in (("fp16", 0, 0, 0), ("tq", 1, 0, 0), ("tiered", 2, 0, 0), ("three_tier", 2, warm_window, 0),
                             ("evicting", 2, warm_window, cool_window)):
        cfg = dict(base, n_layers=1, vocab=1024, batch=1, kv_kind=kind, max_seq=ctx_len + 16 * (steps // 16 + 2),
                   hot_window=hot_window if kind == 2 else 0, warm_window=W, cool_window=C)
        m = nexus_amd.Model(ctx, **cfg)
        m.fill_context(ctx_len, 4 if kind else 0)
        m.decode_untimed(2)
        ctx.sync()
        t0 = time.perf_counter()
        m.decode_untimed(steps)
        ctx.sync()
        step_ms = (time.perf_counter() - t0) * 1e3 / steps
        ms, nb = m.time_attention(200)
        m.close()
        gbs = nb / (ms * 1e-3) / 1e9
        n = ctx_len + 2 + steps  # positions held after the run
        if kind == 0:
            res = n * per["f16"]
        elif kind == 1:
            res = n * per["tq"]
        else:
            cold = 16 * max(0, (n - hot_window) // 16)
            cool = 16 * max(0, (n - hot_window - W) // 16) if W else 0
            evict = 16 * max(0, (n - hot_window - W - C) // 16) if C else 0
            res = (n - cold) * per["f16"] + (cold - cool) * per["tq"] + (cool - evict) * per["cool"]
        out[name] = {"attention_us": round(ms * 1e3, 2), "kv_bytes": int(nb), "GBps": round(gbs, 1),
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "step_ms_1layer": round(step_ms, 4),
                     "resident_bytes": int(res)}
    out["kv_bytes_vs_fp16"] = round(out["tiered"]["kv_bytes"] / out["fp16"]["kv_bytes"], 4)
    return out


def prefill_bench(ctx, base: dict, P: int = 2048) -> dict:
    """Batched prefill throughput of a P-token prompt (fresh model, positions
    from 0) and the TFLOP/s of its gate/up GEMM at the 2048-token chunk."""
    import ctypes as C

    import numpy as np

    import nexus_amd
    cfg = dict(base, batch=1, kv_kind=0, max_seq=((P + 64) // 16 + 1) * 16)
    prompt = np.random.default_rng(1).integers(0, base["vocab"], (1, P), dtype=np.int32)
    m = nexus_amd.Model(ctx, **cfg)
    m.prefill(prompt[:, :64])  # first launches of every kernel
    m.close()
    m = nexus_amd.Model(ctx, **cfg)
    ctx.sync()
    t0 = time.perf_counter()
    m.prefill(prompt)
    ctx.sync()
    dt = time.perf_counter() - t0
    m.close()
    d, F, L = base["d_model"], base["ffn"], base["n_layers"]
    qkv = (base["n_heads"] + 2 * base["n_kv_heads"]) * base["head_dim"]
    # routed experts: each token runs top_k experts' FFNs and the router
    experts = base["top_k"] if base["n_experts"] > 0 else 1
    w_flops = 2.0 * P * L * d * (qkv + base["n_heads"] * base["head_dim"] + 3 * F * experts + base["n_experts"])
    att_flops = 4.0 * L * base["n_heads"] * base["head_dim"] * P * (P + 1) / 2
    M, N, K = 2048, 2 * F, d
    G = (K + 31) // 32
    bx, bw, bs, by = ctx.alloc(M * K * 2), ctx.alloc(N * G * 16), ctx.alloc(N * G * 2), ctx.alloc(M * N * 4)
    ms = C.c_double()
    ctx.check(ctx.L.nx_time_gemm(ctx.h, bx, bw, bs, by, M, N, K, 50, C.byref(ms)), "nx_time_gemm")
    for b in (bx, bw, bs, by):
        ctx.free(b)
    tf = 2.0 * M * N * K / (ms.value * 1e-3) / 1e12
    return {"tokens": P, "ms": round(dt * 1e3, 2), "tok_s": round(P / dt, 1),
            "TFLOPs_end_to_end": round((w_flops + att_flops) / dt / 1e12, 1),
            "roofline": {"kernel": f"k_pf_gemm int4-g32 GEMM, gate/up {N}x{K}, {M}-token chunk", "bound": "mfma",
                         "achieved": round(tf, 1), "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / PEAK_MFMA_TFLOPS, 4), "avg_us": round(ms.value * 1e3, 2)}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--model", choices=sorted(MODELS), default="llama-8b")
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--kv", choices=["fp16", "tq", "tiered"], default="fp16")
    ap.add_argument("--hot-window", type=int, default=4096,
                    help="tiered pages: positions kept fp16 (older pages TurboQuant)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode measurement (no GEMV, NXF, prefill or tiering lines)")
    ap.add_argument("--profile-kernel", choices=["ffn", "attention", "xxh32", "gemv"],
                    help="only launch one kernel 64 times over the layers (for rocprofv3 --pmc); gemv: "
                         "the standalone GEMV microbench of --gemv-shape at --batch")
    ap.add_argument("--gemv-shape", default="14336x4096", help="N x K of --profile-kernel gemv")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the batched prefill measurement (for rocprofv3)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only copy a 256 MiB buffer 16 times (counter calibration kernel)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(--gpus must be 1).", file=sys.stderr)
        return 2
    if args.copy_calib:
        import torch
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(16):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calib_bytes_per_launch_read": src.numel() * 4,
                          "copy_calib_bytes_per_launch_write": dst.numel() * 4, "launches": 16}))
        return 0

    import nexus_amd

    if args.prefill_only:
        ctx = nexus_amd.Context(0)
        print(json.dumps({"prefill": prefill_bench(ctx, MODELS[args.model])}))
        ctx.close()
        return 0
    if args.profile_kernel == "gemv":
        global GEMV_SHAPES
        GEMV_SHAPES = [tuple(int(v) for v in args.gemv_shape.split("x"))]
        ctx = nexus_amd.Context(0)
        for r in gemv_microbench(ctx, args.batch, iters=20):
            print(json.dumps(r))
        ctx.close()
        return 0
    if args.profile_kernel == "xxh32":
        ctx = nexus_amd.Context(0)
        r = nxf_verify_bench(ctx, False, iters=16)
        print(json.dumps({"kernel": "xxh32", "avg_us": r["avg_us"], "bytes": r["bytes"], "launches": 17}))
        ctx.close()
        return 0
    kv_kind = {"fp16": 0, "tq": 1, "tiered": 2}[args.kv]
    smp_steps = max(8, args.steps // 2)  # sampled decode steps after the greedy ones
    max_seq = ((args.ctx + args.warmup + args.steps + smp_steps + 24) // 16 + 1) * 16
    base = MODELS[args.model]
    moe = base["n_experts"] > 0
    cfg = dict(base, batch=args.batch, kv_kind=kv_kind, max_seq=max_seq,
               hot_window=args.hot_window if kv_kind == 2 else 0)
    ctx = nexus_amd.Context(0)
    print(f"[bench] device {ctx.device_name()}; building {args.model}-shaped model "
          f"(batch {args.batch}, ctx {args.ctx}, kv {args.kv})", file=sys.stderr, flush=True)
    model = nexus_amd.Model(ctx, **cfg)
    model.fill_context(args.ctx, 4 if kv_kind else 0)
    model.decode_untimed(1)
    if args.profile_kernel:
        ms, nb = (model.time_ffn_gemv if args.profile_kernel == "ffn" else model.time_attention)(64)
        print(json.dumps({"kernel": args.profile_kernel, "avg_us": round(ms * 1e3, 3),
                          "bytes": int(nb), "launches": 64 + base["n_layers"]}))
        model.close()
        ctx.close()
        return 0
    # the dominant kernel and the attention timed over the filled context
    # (the launches the committed PMC summary of --profile-kernel counts)
    ffn_ms, ffn_bytes = model.time_ffn_gemv(200)
    att_ms, att_bytes = model.time_attention(200)
    if args.warmup > 0:
        model.decode_untimed(args.warmup)
    bytes_start = model.step_bytes()
    ctx.sync()
    t0 = time.perf_counter()
    model.decode_untimed(args.steps)  # launches K step graphs and waits for them
    ctx.sync()
    t1 = time.perf_counter()
    bytes_end = model.step_bytes()
    elapsed = t1 - t0
    tok_s = args.steps * args.batch / elapsed
    step_bytes = 0.5 * (bytes_start + bytes_end)
    print(f"[bench] {args.steps} steps in {elapsed * 1e3:.2f} ms; {step_bytes / 1e9:.3f} GB/step",
          file=sys.stderr, flush=True)

    # the same decode with sampling in the step graph (SamplingParams defaults
    # of core/config.h:60-66 with a fixed seed)
    model.set_sampling(0.7, 40, 0.9, 42)
    model.decode_untimed(2)
    ctx.sync()
    t0 = time.perf_counter()
    model.decode_untimed(smp_steps)
    ctx.sync()
    smp_s = time.perf_counter() - t0
    model.set_sampling(0.0, 0, 1.0, 0)
    sampling = {"params": {"temperature": 0.7, "top_k": 40, "top_p": 0.9, "seed": 42}, "steps": smp_steps,
                "tok_s": round(smp_steps * args.batch / smp_s, 2),
                "ms_per_step": round(smp_s * 1e3 / smp_steps, 4),
                "greedy_ms_per_step": round(elapsed * 1e3 / args.steps, 4)}
    if not args.no_cpu:
        import numpy as np

        import oracle
        lg = np.random.default_rng(2).standard_normal(base["vocab"]).astype(np.float32) * 3
        t0 = time.perf_counter()
        for _ in range(10):
            oracle.lib.nxo_sample(lg, base["vocab"], 0.7, 40, 0.9, 0.5)
        sampling["cpu_ms_per_sample"] = round((time.perf_counter() - t0) * 100, 3)
    ffn_gbs = ffn_bytes / (ffn_ms * 1e-3) / 1e9
    att_gbs = att_bytes / (att_ms * 1e-3) / 1e9
    model.close()
    full = not args.decode_only
    micro = (gemv_microbench(ctx, 1) + gemv_microbench(ctx, 8)) if full and not moe else None
    # the other decode workloads, when the default one is measured
    others = None
    if full and args.model == "llama-8b" and args.batch == 1 and kv_kind == 0 and args.ctx == 4096:
        print("[bench] other decode workloads", file=sys.stderr, flush=True)
        cpu = not args.no_cpu
        others = [
            decode_line(ctx, TINY, "tiny llama (2 layers, d 256), 16-token prompt", 1, 0, 16, 64, prompt=True),
            decode_line(ctx, LLAMA8B, "llama-3.1-8b-shape, fp16 paged KV", 8, 0, 4096, 128, cpu=cpu),
            decode_line(ctx, LLAMA8B, "llama-3.1-8b-shape, TurboQuant 3.5-bit paged KV", 1, 1, 32768, 64, cpu=cpu),
            decode_line(ctx, MIXTRAL, "mixtral-8x7b-shape (top-2 of 8), fp16 paged KV", 1, 0, 4096, 128, cpu=cpu),
            decode_line(ctx, MIXTRAL, "mixtral-8x7b-shape (top-2 of 8), fp16 paged KV", 8, 0, 4096, 128, cpu=cpu),
        ]
    nxf = nxf_verify_bench(ctx, not args.no_cpu) if full else None
    pre = prefill_bench(ctx, base) if full else None
    tier = tiering_bench(ctx, base) if full and base["head_dim"] == 128 else None
    ctx.close()
    kv_name = ["fp16", "TurboQuant 3.5-bit", f"tiered (last {args.hot_window} positions fp16, older pages "
               "TurboQuant 3.5-bit)"][kv_kind]
    if moe:
        workload = (f"mixtral-8x7b-shape int4-g32 greedy decode (top-2 of 8 experts), batch {args.batch}, "
                    f"ctx {args.ctx} {kv_name} paged KV")
        ffn_kernel = "routed gate/up int4-g32 expert GEMV + SwiGLU (active experts x 28672 x 4096)"
    else:
        workload = (f"llama-3.1-8b-shape int4-g32 greedy decode, batch {args.batch}, "
                    f"ctx {args.ctx} {kv_name} paged KV")
        ffn_kernel = "fused RMSNorm + gate/up int4-g32 GEMV + SwiGLU (28672 x 4096)"

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-g32 x fp16 -> fp32 accumulate",
        "data": "synthetic (seeded device generator; random-init weights)",
        "config": {
            "workload": workload,
            "batch": args.batch, "ctx": args.ctx, "layers": base["n_layers"], "d_model": base["d_model"],
            "ffn": base["ffn"], "vocab": base["vocab"], "experts": base["n_experts"], "top_k": base["top_k"],
            "parallelism": "none (1 GPU)",
        },
        "hbm_GBps_end_to_end": round(step_bytes / (elapsed / args.steps) / 1e9, 1),
        "roofline": {
            "kernel": ffn_kernel,
            "bound": "hbm", "achieved": round(ffn_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(ffn_gbs / PEAK_HBM_GBS, 4), "traffic": measured_traffic("ffn", ffn_bytes) if args.batch == 1 else None,
            "avg_us": round(ffn_ms * 1e3, 3), "bytes": int(ffn_bytes),
        },
        "attention": {
            "kernel": "paged decode attention, one layer", "achieved": round(att_gbs, 1),
            "frac": round(att_gbs / PEAK_HBM_GBS, 4), "avg_us": round(att_ms * 1e3, 3),
            "bytes": int(att_bytes), "traffic": ({0: measured_traffic("attention", att_bytes),
                         1: measured_traffic("attention_tq", att_bytes)}.get(kv_kind)
                        if args.batch == 1 and args.model == "llama-8b" else None),
        },
        "roofline_end_to_end_frac": round(step_bytes / (elapsed / args.steps) / 1e9 / PEAK_HBM_GBS, 4),
    }
    if micro is not None:
        line["gemv_microbench"] = micro
    if others is not None:
        line["decode_workloads"] = others
    if nxf is not None:
        line["nxf_verify"] = nxf
    line["sampling"] = sampling
    if pre is not None:
        line["prefill"] = pre
    if tier is not None:
        line["tiering"] = tier
    if not args.no_cpu:
        print("[bench] timing the CPU oracle baseline", file=sys.stderr, flush=True)
        hw = args.hot_window if kv_kind == 2 else 0
        line["cpu_baseline"] = cpu_baseline(base, args.ctx, args.batch, kv_kind, hw)
        line["cpu_baseline"]["cpu_model"] = cpu_model_name()
        if full:
            line["cpu_baselines"] = cpu_baselines(base, args.ctx, args.batch, kv_kind, hw)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

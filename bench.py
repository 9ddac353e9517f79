#!/usr/bin/env python3
"""Decode benchmark: Llama-3.2-1B-shaped bf16 decoder, batch 1, on one MI355X.

Workload (one "step" = one decode token through the whole forward pass):
random-init bf16 weights (seed 0, N(0, 0.02), RMSNorm weights 1) in the
Llama-3.2-1B shape (16 layers, hidden 2048, 32/8 heads, hd 64, SwiGLU 8192,
vocab 128256, tied, interleaved RoPE theta 5e5), a 512-token random prompt
(seed 1), then greedy decode of --steps tokens with a 4096-position f32 KV
cache. Timing follows generateGreedyMeasured (src/generator.zig:221-293):
decode tok/s = generated tokens / decode time; prefill tok/s = prompt tokens /
prefill time.

Prints one JSON line with the headline metric, the roofline of the dominant
kernel (HIP events on the model's stream) and a CPU baseline (the oracle, a
C restatement of the reference CPU path, on a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure
KERNELS = ("qkv", "attention", "o_proj", "gate_up", "down")


def kernel_bytes(cfg, pos: int) -> dict:
    """Algorithmic HBM bytes per launch of each decode kernel at position pos
    (weights read once, activations read/written once)."""
    H, I, V, kv = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.kv_dim()
    T = pos + 1
    bias = (H + 2 * kv) * 2 if cfg.qkv_bias else 0
    # MoE: the top-k experts' gate/up and down (I per expert), the router and
    # the QK-norm weights.
    K = cfg.num_experts_per_token if cfg.num_experts else 1
    router = cfg.num_experts * H * 2 if cfg.num_experts else 0
    qkn = (H + kv) * 2 if cfg.num_experts and cfg.qk_norm else 0
    return {
        "qkv": (H * H + 2 * kv * H) * 2 + bias + H * 2 + H * 4 + (H + 2 * kv) * 4,
        "attention": 2 * T * kv * 4 + 2 * kv * 4 + (H + 2 * kv) * 4 + H * 4 + qkn,
        "o_proj": H * H * 2 + H * 4 + 2 * H * 4,
        "gate_up": K * 2 * I * H * 2 + router + H * 2 + H * 4 + K * I * 4,
        "down": K * H * I * 2 + K * I * 4 + 2 * H * 4,
        "logits": V * H * 2 + H * 2 + H * 4 + V * 4,
    }


def token_bytes(cfg, pos: int) -> int:
    """B(pos): weight bytes of one decode token plus f32 KV read (0..pos) and
    write (pos), the roofline numerator of the headline target."""
    kb = kernel_bytes(cfg, pos)
    L = cfg.num_hidden_layers
    return L * sum(kb[k] for k in KERNELS) + kb["logits"] + cfg.hidden_size * 2


def profile_kernels(runner, cfg, token: int, pos: int, reps: int = 3) -> dict:
    import ctypes

    from vvli_amd import _lib

    L = cfg.num_hidden_layers
    n = 1 + 5 * L + 2
    buf = (ctypes.c_float * n)()
    got = ctypes.c_uint32()
    acc = np.zeros(n)
    for _ in range(reps):
        _lib.check(_lib.lib().vvli_gpu_profile_step(runner._h, token, pos, buf, n, ctypes.byref(got)))
        acc += np.frombuffer(buf, dtype=np.float32)[: got.value]
    ms = acc / reps
    out = {"embed": [ms[0]], "logits": [ms[1 + 5 * L]], "argmax": [ms[2 + 5 * L]]}
    for i, k in enumerate(KERNELS):
        out[k] = [ms[1 + 5 * l + i] for l in range(L)]
    return out


def measured_traffic(symbol: str, model: str):
    """The committed rocprofv3 PMC measurement of `symbol` on `model`
    (FETCH_SIZE + WRITE_SIZE of one launch, calibrated on a 256 MiB copy):
    dict(traffic, algorithmic, steps, pos) -- the launch's measured HBM bytes,
    its algorithmic bytes, and the decode steps / first position it ran -- or
    None where no summary covers that kernel and workload."""
    path = ROOT / "profiles" / "pmc_traffic_llama1b_decode.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.strip().split("\t")
        if len(parts) == 7 and parts[0] == "traffic" and parts[1] == symbol and parts[2] == model:
            return {"traffic": int(parts[3]), "algorithmic": int(parts[4]), "steps": int(parts[5]),
                    "pos": int(parts[6])}
    return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(cfg, blob, prompt, budget_s: float, max_tokens: int, inv_freq=None) -> dict:
    """Decode tok/s of the oracle (C restatement of the reference CPU path:
    per-call thread fan-out over rows, single-threaded attention) on this
    host, at the positions the GPU decodes: the prompt goes through the
    oracle's prompt pass (bit-identical to its token loop, untimed), then
    greedy decode steps are timed for about budget_s seconds."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = oracle.cpu_count()
    r = oracle.OracleRunner(cfg, blob, len(prompt) + max_tokens + 16, threads=threads, lanes=16)
    if inv_freq is not None:
        r.set_rope_table(inv_freq)
    t0 = time.perf_counter()
    logits = r.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    tokens = []
    t0 = time.perf_counter()
    pos = len(prompt)
    while len(tokens) < max_tokens and (time.perf_counter() - t0) < budget_s:
        nxt = oracle.argmax(logits)
        tokens.append(nxt)
        logits = r.forward_token(nxt, pos)
        pos += 1
    dt = time.perf_counter() - t0
    r.close()
    return {"tokens": tokens, "seconds": dt, "threads": threads, "prefill_s": prefill_s}


def open_runner(args, cfg, blob):
    """The decode runner over blob: uploaded directly (--source synthetic) or
    written as a bf16 GGUF file and loaded through the device GGUF loader
    (mmap -> HBM, vvli_gpu_model_create_from_gguf), the form the Llama-3.2-1B
    workload specifies. Returns (runner, description of the source)."""
    from vvli_amd import runtime as R

    if args.source != "gguf":
        return R.Runner(cfg, blob, args.ctx), "synthetic blob uploaded from host memory"
    import tempfile

    from vvli_amd import gguf_write
    from vvli_amd import loaders as L

    tmpd = tempfile.mkdtemp(prefix="vvli_bench_")
    path = os.path.join(tmpd, f"{args.model}.gguf")
    try:
        t = time.perf_counter()
        size = gguf_write.write_dense_gguf(path, cfg, blob)
        tw = time.perf_counter() - t
        t = time.perf_counter()
        gcfg, runner = L.device_load_gguf(path, args.ctx)
        tl = time.perf_counter() - t
    finally:
        if os.path.exists(path):
            os.remove(path)
        os.rmdir(tmpd)
    for f in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
              "num_key_value_heads", "tie_word_embeddings", "rope_layout"):
        if getattr(gcfg, f) != getattr(cfg, f):
            raise RuntimeError(f"GGUF round trip changed {f}: {getattr(gcfg, f)} != {getattr(cfg, f)}")
    print(f"[bench] bf16 GGUF {size / 1e9:.2f} GB written in {tw:.1f}s, loaded to the device in {tl:.1f}s",
          file=sys.stderr, flush=True)
    return runner, f"bf16 GGUF file ({size / 1e9:.2f} GB) through the device GGUF loader (mmap -> HBM)"


def gemv_sweep(shapes, ms, log=True) -> list:
    """vvli_gpu_linear over (N, K) x M: bf16 W [N, K] ~ N(0, 0.02), f32 X [M, K]
    ~ N(0, 1), f32 Y [M, N]. Each shape rotates over enough weight copies
    (>= 1 GiB) that W is read from HBM, not from the 256 MB memory-side cache.
    Algorithmic bytes 2NK + 4MK + 4MN, flops 2MNK.

    Time per call, two ways: `us` -- a HIP graph of `reps` back-to-back calls
    (one per weight copy in turn), HIP events around its replay, so the GPU
    runs the kernels back to back without waiting for the host (the op's
    device time including the gap between launches; the median of five
    replays); `us_host_loop` -- the
    same calls issued one by one from Python through ctypes, HIP events
    around the loop (bounded below by the host's per-call cost, about 3 us
    here). The graph is captured on a stream whose scratch the warm-up calls
    already sized, so the capture records kernels only."""
    import torch

    from vvli_amd import runtime as R

    gen = torch.Generator(device="cuda").manual_seed(0)
    stream = torch.cuda.Stream()
    rows = []
    for n, k in shapes:
        wbytes = 2 * n * k
        copies = max(2, -(-(1 << 30) // wbytes))
        ws = [(torch.randn(n, k, device="cuda", generator=gen) * 0.02).to(torch.bfloat16) for _ in range(copies)]
        for m in ms:
            x = torch.randn(m, k, device="cuda", generator=gen)
            y = torch.empty(m, n, device="cuda")
            reps = max(copies, 20)
            torch.cuda.synchronize()

            def call(i):
                R.linear(ws[i % copies].data_ptr(), x.data_ptr(), y.data_ptr(), m, n, k, stream=stream.cuda_stream)

            with torch.cuda.stream(stream):
                for i in range(3):
                    call(i)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for i in range(reps):
                    call(i)
                e1.record(stream)
            e1.synchronize()
            us_host = e0.elapsed_time(e1) * 1e3 / reps
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(reps):
                    call(i)
            samples = []
            with torch.cuda.stream(stream):
                g.replay()
                stream.synchronize()
                for _ in range(5):  # the median of five timed replays: one slow replay does not set the figure
                    e0.record(stream)
                    g.replay()
                    e1.record(stream)
                    e1.synchronize()
                    samples.append(e0.elapsed_time(e1) * 1e3 / reps)
            us = sorted(samples)[len(samples) // 2]
            del g
            nbytes = 2 * n * k + 4 * m * k + 4 * m * n
            rows.append({"N": n, "K": k, "M": m, "us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1),
                         "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                         "tflops": round(2 * m * n * k / us / 1e6, 1), "us_host_loop": round(us_host, 2)})
            if log:
                print(f"[bench] linear N={n} K={k} M={m}: {us:.2f} us (graph), {nbytes / us / 1e3:.0f} GB/s, "
                      f"{2 * m * n * k / us / 1e6:.1f} TFLOP/s; host loop {us_host:.2f} us", file=sys.stderr,
                      flush=True)
        del ws
        torch.cuda.empty_cache()
    return rows


LINEAR_SHAPES = [(2048, 2048), (512, 2048), (8192, 2048), (2048, 8192), (128256, 2048)]


PHASE_KINDS = ("Q", "A", "O", "G", "D")
PHASE_BYTES = {"Q": "qkv", "A": "attention", "O": "o_proj", "G": "gate_up", "D": "down"}


def phases_main(args, cfg, blob) -> int:
    """Per-phase critical path of the persistent decode step
    (vvli_gpu_profile_persistent, s_memrealtime marks at 100 MHz): after a
    batched prefill of --prompt tokens, one profiled step at every position of
    the decode range. A phase's time is the end of its last wave minus the end
    of the previous phase's last wave; `staged` is when the median block had
    its input in LDS, measured from that same previous end (the hop). Bytes per
    phase are the algorithmic bytes of the matching per-kernel launch
    (kernel_bytes) at the step's position."""
    import ctypes

    from vvli_amd import _lib
    from vvli_amd import runtime as R

    runner = (R.MoeRunner if cfg.num_experts else R.Runner)(cfg, blob, args.ctx)
    runner.set_decode_path("persistent")
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, size=args.prompt).astype(np.uint32)
    runner.prefill(prompt)
    L = cfg.num_hidden_layers
    NP = 5 * L + 2
    S = 16
    stride = S * NP
    nb = ctypes.c_uint32()
    buf = np.zeros((1024 + 1) * stride, dtype=np.uint64)
    positions = list(range(args.prompt, args.prompt + args.steps))
    dur = {k: [] for k in PHASE_KINDS + ("logits",)}
    hop = {k: [] for k in PHASE_KINDS + ("logits",)}
    gbs = {k: [] for k in PHASE_KINDS + ("logits",)}
    step_us = []
    moe_marks = {"route": [], "publish": [], "last_pub": [], "after_last": []}  # MoE gate/up: slots 14, 15
    stg = {k: {"begin": [], "first": [], "retries": [], "own": [], "bar": [], "pre": []} for k in PHASE_KINDS + ("logits",)}
    attn = {k: [] for k in ("q", "pass", "partials stored", "partials polled", "weights", "published")}
    for pos in positions:
        buf[:] = 0
        _lib.check(_lib.lib().vvli_gpu_profile_persistent(runner._h, 5, pos, ctypes.c_void_p(buf.ctypes.data), stride,
                                                          ctypes.byref(nb)))
        n = nb.value
        t = buf[: (n + 1) * stride].reshape(n + 1, NP, S).astype(np.int64)
        prev = t[n, 0, 0]  # kernel start
        start = prev
        kb = kernel_bytes(cfg, pos)
        for ph in range(5 * L + 1):
            kind = "logits" if ph == 5 * L else PHASE_KINDS[ph % 5]
            ends = t[:n, ph, 1:9]
            end = ends[ends > 0].max()
            st = t[:n, ph, 0]
            st = st[st > 0]
            ent, fst, rty = t[:n, ph, 9], t[:n, ph, 10], t[:n, ph, 11]
            okb = (ent > 0) & (fst > 0)
            if kind == "A":  # attention units: their own marks (slots 9, 10, 11, 14, 15, 0), no input staging
                unit = t[:n, ph, 9] > 0
                for key, sl in (("q", 9), ("pass", 10), ("partials stored", 11), ("partials polled", 14),
                                ("weights", 15), ("published", 0)):
                    v = t[:n, ph, sl][unit]
                    attn[key] += list((v[v > 0] - prev) * 1e-2)
                st = np.zeros(0)
                okb = np.zeros_like(okb)
            if okb.any():  # thread 0 of each staging block: entry after the previous end, first attempt, retries
                stg[kind]["begin"] += list((ent[okb] - prev) * 1e-2)
                stg[kind]["first"] += list((fst[okb] - ent[okb]) * 1e-2)
                stg[kind]["retries"] += list(rty[okb])
                if ph > 0:  # entry after the block's own last wave of the previous phase
                    own = t[:n, ph - 1, 1:9].max(axis=1)
                    sel = okb & (own > 0)
                    stg[kind]["own"] += list((ent[sel] - own[sel]) * 1e-2)
                    bar, pre = t[:n, ph - 1, 12], t[:n, ph - 1, 13]
                    sel2 = sel & (bar > 0) & (pre > 0)
                    stg[kind]["bar"] += list((bar[sel2] - own[sel2]) * 1e-2)  # closing barrier
                    stg[kind]["pre"] += list((pre[sel2] - bar[sel2]) * 1e-2)  # the end-of-phase marks (MoE: the router row prefetch)
            if cfg.num_experts and kind == "G":
                s0, s14, s15 = t[:n, ph, 0], t[:n, ph, 14], t[:n, ph, 15]
                sel = (s0 > 0) & (s14 > 0)
                moe_marks["route"] += list((s14[sel] - s0[sel]) * 1e-2)
                pr = (s0 > 0) & (s15 > 0)
                if pr.any():
                    moe_marks["publish"] += list((s15[pr] - s0[pr]) * 1e-2)
                    moe_marks["last_pub"].append((s15[pr].max() - np.median(s0[s0 > 0])) * 1e-2)
                    moe_marks["after_last"] += list((s14[sel] - s15[pr].max()) * 1e-2)
            us = (end - prev) * 1e-2
            dur[kind].append(us)
            hop[kind].append((np.median(st) - prev) * 1e-2 if st.size else np.nan)
            gbs[kind].append(kb[PHASE_BYTES.get(kind, "logits")] / (us * 1e-6) / 1e9)
            prev = end
        step_us.append((prev - start) * 1e-2)
    rows = {}
    for k in PHASE_KINDS + ("logits",):
        per = 1 if k == "logits" else L
        b = kernel_bytes(cfg, positions[len(positions) // 2])[PHASE_BYTES.get(k, "logits")]
        hk = [h for h in hop[k] if not np.isnan(h)]  # (the attention phase stages nothing)
        rows[k] = {"us": round(float(np.median(dur[k])), 2), "hop_us": round(float(np.median(hk)), 2) if hk else None,
                   "bytes": int(b), "gbs": round(float(np.median(gbs[k])), 1), "per_token": per,
                   "us_per_token": round(float(np.median(dur[k])) * per, 1)}
    names = {"Q": "q/k/v (RMSNorm + GEMV + bias)", "A": "attention (RoPE, KV append, split merge)",
             "O": "o_proj + residual", "G": "gate/up + SwiGLU", "D": "down + residual",
             **({"A": "attention (QK-norm, RoPE, KV append, split merge)",
                 "G": "router + top-k + experts' gate/up + SwiGLU",
                 "D": "experts' down + weighted sum + residual"} if cfg.num_experts else {}),
             "logits": "final RMSNorm + lm_head + argmax keys"}
    md = ["| phase | median us | staged after (us) | algorithmic bytes | GB/s | % of 8 TB/s | per token | us per token |",
          "|---|---|---|---|---|---|---|---|"]
    for k, r in rows.items():
        hop_s = f"{r['hop_us']:.2f}" if r["hop_us"] is not None else "-"
        md.append(f"| {names[k]} | {r['us']:.2f} | {hop_s} | {r['bytes']:,} | {r['gbs']:.0f} | "
                  f"{100 * r['gbs'] / HBM_PEAK_GBS:.1f} | x{r['per_token']} | {r['us_per_token']:.1f} |")
    med_step = float(np.median(step_us))
    md.append(f"| whole step (kernel start to logits end) | {med_step:.1f} | | "
              f"{token_bytes(cfg, positions[len(positions) // 2]):,} | "
              f"{token_bytes(cfg, positions[len(positions) // 2]) / med_step / 1e3:.0f} | "
              f"{100 * token_bytes(cfg, positions[len(positions) // 2]) / med_step / 1e3 / HBM_PEAK_GBS:.1f} | | |")
    print("\n".join(md), file=sys.stderr, flush=True)
    if cfg.num_experts and moe_marks["route"]:
        r = np.array(moe_marks["route"])
        print(f"[bench] MoE gate/up: routed p50 {np.median(r):.2f} p90 {np.percentile(r, 90):.2f} us after the "
              f"staged input; router row published p50 {np.median(moe_marks['publish']):.2f} us after a producer's "
              f"staged input, the last one p50 {np.median(moe_marks['last_pub']):.2f} us after the median block's; "
              f"routed p50 {np.median(moe_marks['after_last']):.2f} us after the last publication",
              file=sys.stderr, flush=True)
    if attn["q"]:
        print("[bench] attention units, us after the q/k/v phase's end (p50): " +
              ", ".join(f"{k} {np.median(v):.2f}" for k, v in attn.items() if v), file=sys.stderr, flush=True)
    for k in PHASE_KINDS + ("logits",):
        d = stg[k]
        if d["begin"]:
            b, f, r = np.array(d["begin"]), np.array(d["first"]), np.array(d["retries"])
            print(f"[bench] staging {k}: entry after prev end p50 {np.median(b):.2f} p90 {np.percentile(b, 90):.2f} "
                  f"max {b.max():.2f} us; first attempt p50 {np.median(f):.2f} p90 {np.percentile(f, 90):.2f} us; "
                  f"retries p50 {np.median(r):.0f} p90 {np.percentile(r, 90):.0f} max {r.max():.0f}"
                  + (f"; entry after the block's own previous end p50 {np.median(d['own']):.2f} "
                     f"p90 {np.percentile(d['own'], 90):.2f} max {np.max(d['own']):.2f} us" if d["own"] else "")
                  + (f" = barrier p50 {np.median(d['bar']):.2f} + {np.median(d['pre']):.2f} to the set-up of the next phase + rest"
                     if d["bar"] else ""),
                  file=sys.stderr, flush=True)
    line = {"metric": "persistent decode step: per-phase critical path", "value": round(med_step, 1), "unit": "us",
            "n_gpus": 1, "steps": len(positions), "warmup": 0, "ms_per_step": round(med_step / 1e3, 4),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": f"{args.model} bf16 decode step, profiled at pos {positions[0]}-{positions[-1]}",
                       "ctx": args.ctx}, "phases": rows, "cpu_baseline": None}
    print(json.dumps(line), flush=True)
    runner.close()
    return 0


def make_blob(cfg):
    """Seeded synthetic bf16 weights: N(0, 0.02), RMSNorm weights 1; MoE
    routers N(0, 1/sqrt(hidden)) so router logits are about N(0, 1)."""
    from vvli_amd import config as C
    from vvli_amd import runtime as R

    blob = R.synthetic_blob(cfg, C.WEIGHT_BF16, seed=0, stddev=0.02)
    if cfg.num_experts:
        n = cfg.num_experts * cfg.hidden_size
        rng = np.random.default_rng(100)
        for l in range(cfg.num_hidden_layers):
            off = R.moe_slice_offset(cfg, l, "router")
            v = rng.normal(0, 1 / np.sqrt(cfg.hidden_size), n).astype(np.float32).view(np.uint32).astype(np.uint64)
            blob[off:off + n] = ((v + 0x7FFF + ((v >> 16) & 1)) >> 16).astype(np.uint16)
    return blob


def moe_token_bytes(cfg, pos: int) -> int:
    """Algorithmic HBM bytes of one MoE decode token: attention weights, the
    router, the top-k experts' gate/up/down, norms, lm_head, the embedding row
    and the f32 KV read (0..pos) and write."""
    H, I, V, kv = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.kv_dim()
    E, K, L = cfg.num_experts, cfg.num_experts_per_token, cfg.num_hidden_layers
    layer = 2 * (H * H * 2 + 2 * kv * H) + 2 * (2 * H + (H + kv if cfg.qk_norm else 0))
    layer += E * H * 2 + K * 3 * I * H * 2
    kv_bytes = L * 2 * kv * 4 * (pos + 2)
    return L * layer + V * H * 2 + H * 2 + H * 2 + kv_bytes


def moe_decode_main(args, cfg, blob) -> int:
    """MoE decode (per-kernel graph path): tok/s and the whole-step roofline."""
    import torch

    from vvli_amd import runtime as R

    runner = R.MoeRunner(cfg, blob, args.ctx)
    runner.set_decode_path(args.path)
    persistent = args.path == "persistent" or (args.path == "auto" and runner.persistent_available())
    batched = args.prefill == "batched"
    runner.set_prefill_path("auto" if batched else "loop")
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, size=args.prompt).astype(np.uint32)
    runner.generate_greedy_measured(prompt[:8], max(1, args.warmup), batched_prefill=batched)
    runner.kv_clear()
    torch.cuda.synchronize()
    _, stats = runner.generate_greedy_measured(prompt, args.steps, batched_prefill=batched)
    torch.cuda.synchronize()
    decode_s = stats.decode_nanoseconds / 1e9
    tok_s = args.steps / decode_s
    step_bytes = sum(moe_token_bytes(cfg, p) for p in range(args.prompt, args.prompt + args.steps))
    gbs = step_bytes / decode_s / 1e9
    line = {
        "metric": "decode tok/s @bs1 + HBM GB/s (% of peak), MoE", "value": round(tok_s, 2), "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(decode_s * 1e3 / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{args.model} bf16 greedy decode, bs1", "prompt_tokens": args.prompt,
                   "decode_tokens": args.steps, "ctx": args.ctx, "kv_cache": "f32", "parallelism": "none (1 GPU)"},
        "prefill_tok_s": round(stats.prefill_tokens_per_second(), 2),
        "prefill": "batched (grouped expert GEMMs)" if batched else "token loop",
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": ("MoE persistent decode step (one cooperative launch for the decode loop)"
                                if persistent else "MoE token step (per-kernel HIP graph, one replay per token)"),
                     "bytes_per_launch": step_bytes // args.steps},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    runner.close()
    return 0


def prefill_main(args, cfg, blob) -> int:
    """Batched-prefill sweep (vvli_gpu_prefill): best of three per length.
    Flops = 2 * rows * (projection weights) + 4 * heads * hd * (causal key
    count) per layer: the useful work, without the lo half of the hi/lo split."""
    import torch

    from vvli_amd import runtime as R

    runner = R.Runner(cfg, blob, args.ctx)
    runner.set_prefill_path("batched")
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, size=args.ctx).astype(np.uint32)
    runner.prefill(prompt[:64])
    H, I, kv, L = cfg.hidden_size, cfg.intermediate_size, cfg.kv_dim(), cfg.num_hidden_layers
    proj = L * (H * H + 2 * kv * H + H * H + 3 * I * H)

    def flops(n):
        return 2 * n * proj + L * 4 * cfg.num_attention_heads * cfg.head_dim() * n * (n + 1) // 2

    sweep = {}
    lengths = {int(v) for v in args.prefill_sweep.split(",")} if args.prefill_sweep else \
        {128, 512, 2048, min(4096, args.ctx)}
    for n in sorted(lengths | {args.prompt}):
        if n > args.ctx:
            continue
        best = 1e9
        for _ in range(3):
            runner.kv_clear()
            torch.cuda.synchronize()
            t = time.perf_counter()
            runner.prefill(prompt[:n])
            best = min(best, time.perf_counter() - t)
        sweep[n] = {"ms": round(best * 1e3, 3), "tok_s": round(n / best, 1),
                    "tflops": round(flops(n) / best / 1e12, 1)}
        print(f"[bench] prefill n={n}: {best * 1e3:.2f} ms, {n / best:.0f} tok/s", file=sys.stderr, flush=True)
    main_n = args.prompt
    res = sweep[main_n]
    line = {
        "metric": "prefill tok/s (batched), bf16", "value": res["tok_s"], "unit": "tok/s", "n_gpus": 1,
        "steps": 3, "warmup": 1, "ms_per_step": res["ms"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{args.model} bf16 prefill of {main_n} tokens", "ctx": args.ctx},
        "roofline": {"bound": "mfma", "achieved": res["tflops"], "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(res["tflops"] / 2500.0, 4), "traffic": None,
                     "kernel": "whole prefill (GEMMs + attention), wall clock"},
        "sweep": sweep,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    runner.close()
    return 0


def sampled_main(args, cfg, blob) -> int:
    """Sampled decode (vvli_gpu_generate with generator.Options defaults:
    temperature 0.8, top-k 40, top-p 0.95, repeat penalty 1.1 over 64 tokens):
    the whole-token roofline of the greedy benchmark over the same prompt and
    steps; --path picks the decode implementation."""
    from vvli_amd import runtime as R

    runner = R.Runner(cfg, blob, args.ctx)
    runner.set_decode_path(args.path)
    runner.set_prefill_path("auto")
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, size=args.prompt).astype(np.uint32)
    opts = R.Sampling(seed=7, top_k=args.top_k)
    runner.generate(prompt[:16], max(1, args.warmup), opts, batched_prefill=True)
    runner.kv_clear()
    tokens, stats = runner.generate(prompt, args.steps, opts, batched_prefill=True)
    assert stats.generated_tokens == args.steps
    decode_s = stats.decode_nanoseconds / 1e9
    tok_s = args.steps / decode_s
    step_bytes = sum(token_bytes(cfg, p) for p in range(args.prompt, args.prompt + args.steps))
    gbs = step_bytes / decode_s / 1e9
    path = "persistent" if args.path != "graph" and runner.persistent_available() else "graph"
    print(f"[bench] sampled decode {tok_s:.1f} tok/s ({path})", file=sys.stderr, flush=True)
    line = {
        "metric": f"decode tok/s @bs1, sampled (T 0.8, top-k {args.top_k}, top-p 0.95, repeat penalty 1.1)",
        "value": round(tok_s, 2),
        "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(decode_s * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{args.model} bf16 sampled decode, bs1", "prompt_tokens": args.prompt,
                   "decode_tokens": args.steps, "ctx": args.ctx, "path": path},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(gbs / 8000.0, 4), "traffic": None,
                     "kernel": "whole token (step + sampler), wall clock"},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    runner.close()
    return 0


def linear_main(args) -> int:
    """Isolated op sweep (vvli_gpu_linear) on the Llama-3.2-1B projection shapes
    at M in {1, 4, 16, 128, 512} (gemv_sweep)."""
    ms = [int(v) for v in args.linear_m.split(",")]
    rows = gemv_sweep(LINEAR_SHAPES, ms)
    gemv = [r for r in rows if r["M"] == 1] or rows
    agg = sum(2 * r["N"] * r["K"] + 4 * r["K"] * r["M"] + 4 * r["N"] * r["M"] for r in gemv) / sum(r["us"] for r in gemv) / 1e3
    if args.copy_calibration:  # a 256 MiB device copy: the HBM-counter calibration of rocprofv3 --pmc runs
        import torch

        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
    line = {
        "metric": f"linear op sweep: GEMV HBM GB/s (M={gemv[0]['M']}, all five shapes)", "value": round(agg, 1),
        "unit": "GB/s",
        "n_gpus": 1, "steps": len(rows), "warmup": 3, "ms_per_step": None, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 weights, f32 activations", "data": "synthetic",
        "config": {"workload": f"Llama-3.2-1B projection shapes x M in {{{', '.join(map(str, ms))}}}, cold weights",
                   "timing": "HIP graph of back-to-back calls per shape and M (us); Python host loop (us_host_loop)"},
        "roofline": {"bound": "hbm", "achieved": round(agg, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(agg / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "vvli_gpu_linear, M = 1"},
        "sweep": rows, "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="decode tokens timed")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode tokens before the timed run")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU-baseline decode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-gemv-sweep", action="store_true", help="decode mode: skip the M = 1 op sweep")
    ap.add_argument("--linear-m", default="1,4,16,128,512", help="linear mode: comma-separated M values")
    ap.add_argument("--prefill-sweep", default=None,
                    help="prefill mode: comma-separated prompt lengths (default 128,512,2048,4096)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed run, copy a 256 MiB device buffer (HBM-counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--prefill", default="batched", choices=["batched", "loop"],
                    help="prompt processing: batched GEMM prefill, or one token step per prompt token (the reference's loop)")
    ap.add_argument("--mode", default="decode", choices=["decode", "prefill", "linear", "phases"],
                    help="decode: the headline decode benchmark; prefill: batched-prefill throughput sweep; "
                         "linear: the isolated op sweep (vvli_gpu_linear); phases: per-phase timing of the "
                         "persistent decode step")
    ap.add_argument("--model", default="llama-3.2-1b",
                    choices=["llama-3.2-1b", "qwen2.5-0.5b", "qwen2.5-7b", "olmoe-1b-7b"],
                    help="decoder shape (synthetic bf16 weights); the default is the headline workload")
    ap.add_argument("--sampling", action="store_true",
                    help="decode mode: sample with the generator's default options instead of greedy")
    ap.add_argument("--top-k", type=int, default=40, help="--sampling: top_k (0: every finite candidate)")
    ap.add_argument("--source", default=None, choices=["gguf", "synthetic"],
                    help="decode mode: weights through a bf16 GGUF file and the device loader (default for "
                         "llama-3.2-1b, the workload's form) or uploaded from the synthetic host blob")
    ap.add_argument("--rope", default=None, choices=["llama3", "base"],
                    help="decode mode: llama3-scaled RoPE table (default for llama-3.2-1b) or plain theta")
    ap.add_argument("--path", default="auto", choices=["auto", "graph", "persistent"],
                    help="decode implementation: one persistent launch per step (auto) or per-kernel HIP graph")
    args = ap.parse_args()
    llama = args.model == "llama-3.2-1b"
    args.source = args.source or ("gguf" if llama else "synthetic")
    args.rope = args.rope or ("llama3" if llama else "base")

    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported (multi-GPU sharding is not built)",
              file=sys.stderr)
        return 2

    import torch

    from vvli_amd import config as C
    from vvli_amd import runtime as R

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    torch.cuda.set_device(0)
    if args.mode == "linear":
        return linear_main(args)
    cfg = C.NAMED[args.model]()
    t = time.perf_counter()
    blob = make_blob(cfg)
    print(f"[bench] synthetic blob {blob.nbytes / 1e9:.2f} GB in {time.perf_counter() - t:.1f}s", file=sys.stderr,
          flush=True)
    if args.mode == "prefill":
        return prefill_main(args, cfg, blob)
    if args.mode == "phases":
        return phases_main(args, cfg, blob)
    if cfg.num_experts:
        return moe_decode_main(args, cfg, blob)
    if args.sampling:
        return sampled_main(args, cfg, blob)
    runner, source = open_runner(args, cfg, blob)
    inv_freq = None
    if args.rope == "llama3":  # Llama-3.2's rope_scaling: factor 32, low/high freq factors 1 / 4, original ctx 8192
        inv_freq = R.llama3_inv_freq(cfg.head_dim(), cfg.rope_theta)
        runner.set_rope_table(inv_freq)
    runner.set_decode_path(args.path)
    runner.set_prefill_path("auto" if args.prefill == "batched" else "loop")
    batched = args.prefill == "batched"
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, size=args.prompt).astype(np.uint32)

    # Warmup: graph capture, clocks, caches.
    runner.generate_greedy_measured(prompt[:16], max(1, args.warmup), batched_prefill=batched)
    runner.kv_clear()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tokens, stats = runner.generate_greedy_measured(prompt, args.steps, batched_prefill=batched)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    persistent = args.path != "graph" and runner.persistent_available()
    decode_launch_ms = runner.last_launch_ms() if persistent else None
    assert stats.generated_tokens == args.steps
    decode_s = stats.decode_nanoseconds / 1e9
    tok_s = args.steps / decode_s
    prefill_tok_s = stats.prefill_tokens_per_second()
    print(f"[bench] decode {tok_s:.1f} tok/s, prefill {prefill_tok_s:.1f} tok/s (wall {wall:.2f}s)", file=sys.stderr,
          flush=True)

    # Whole-token roofline: sum of B(pos) over the decode positions / decode time.
    positions = range(args.prompt, args.prompt + args.steps)
    step_bytes = sum(token_bytes(cfg, p) for p in positions)
    step_gbs = step_bytes / decode_s / 1e9

    # Per-kernel durations of the per-kernel path, mid-decode: start/stop
    # events at each kernel's own dispatch boundaries on the model's stream
    # (vvli_gpu_profile_step), the same interval a kernel trace reports.
    # Grouped by kernel symbol.
    mid = args.prompt + args.steps // 2
    prof = profile_kernels(runner, cfg, int(tokens[args.steps // 2]), mid)
    kb = kernel_bytes(cfg, mid)
    L = cfg.num_hidden_layers
    groups = {  # kernel symbol -> (step kernels it runs, launches per step)
        "gemv_kernel<bf16, 0> (qkv)": (["qkv"], L),
        "attn_decode_kernel<64> (attention)": (["attention"], L),
        "gemv_kernel<bf16, 1> (o_proj + down)": (["o_proj", "down"], 2 * L),
        "gemv_kernel<bf16, 2> (gate_up)": (["gate_up"], L),
        "gemv_kernel<bf16, 3> (logits)": (["logits"], 1),
    }
    kernels = {}
    for sym, (parts, launches) in groups.items():
        total_ms = float(sum(np.sum(prof[k]) for k in parts))
        nbytes = sum(kb[k] * len(prof[k]) for k in parts)
        kernels[sym] = {"launches": launches, "total_us": total_ms * 1e3, "avg_us": total_ms * 1e3 / launches,
                        "bytes_per_launch": nbytes // launches, "gbs": nbytes / (total_ms * 1e-3) / 1e9}
    if persistent:
        # The persistent decode step is the one kernel of the timed region: its
        # decode launch runs all --steps tokens. Algorithmic bytes per launch =
        # sum over the decode positions of B(pos); duration = HIP events around
        # that launch on the model's stream.
        hd = cfg.head_dim()
        tmpl = f"{64 if hd <= 64 else 128}, {'true' if hd in (64, 128) else 'false'}"
        sym = f"decode_step_kernel<{tmpl}> (persistent decode step)"
        kernels = {sym: {"launches": 1, "total_us": decode_launch_ms * 1e3, "avg_us": decode_launch_ms * 1e3,
                         "bytes_per_launch": step_bytes, "gbs": step_bytes / (decode_launch_ms * 1e-3) / 1e9}}
    dom = max(kernels, key=lambda k: kernels[k]["total_us"])
    d = kernels[dom]
    # HBM bytes of this launch from the committed PMC measurement of the same
    # kernel and workload: its measured / algorithmic ratio applied to this
    # launch's algorithmic bytes (the raw figure when the steps and positions
    # are the profiled ones).
    prof_traffic = measured_traffic(dom.split(" (")[0], args.model)
    traffic, traffic_src = None, None
    if prof_traffic and persistent:
        ratio = prof_traffic["traffic"] / prof_traffic["algorithmic"]
        same = prof_traffic["steps"] == args.steps and prof_traffic["pos"] == args.prompt
        traffic = prof_traffic["traffic"] if same else int(round(ratio * d["bytes_per_launch"]))
        traffic_src = (f"profiles/pmc_traffic_llama1b_decode.md: FETCH_SIZE + WRITE_SIZE of the decode launch "
                       f"over {prof_traffic['steps']} steps at pos {prof_traffic['pos']}-"
                       f"{prof_traffic['pos'] + prof_traffic['steps'] - 1}, {ratio:.3f} x its algorithmic bytes"
                       + ("" if same else "; scaled to this launch's algorithmic bytes"))
    roofline = {"bound": "hbm", "achieved": round(d["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(d["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": dom,
                "bytes_per_launch": d["bytes_per_launch"], "avg_launch_us": round(d["avg_us"], 2),
                "launches_per_step": d["launches"]}
    if traffic_src:
        roofline["traffic_ratio"] = round(traffic / d["bytes_per_launch"], 4)
        roofline["traffic_source"] = traffic_src
    if persistent:
        roofline["tokens_per_launch"] = args.steps
        roofline["us_per_token"] = round(d["avg_us"] / args.steps, 2)
    print("[bench] kernels: " + ", ".join(f"{k} {v['avg_us']:.1f}us {v['gbs']:.0f}GB/s" for k, v in kernels.items()),
          file=sys.stderr, flush=True)

    if args.copy_calibration:
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1.0)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()

    # The drop-in forwardToken boundary as a per-token caller drives it (one
    # call per token, synchronous; the 4 * vocab-byte logits copied into the
    # caller's buffer, or returned as the borrowed view of the library's
    # pinned copy -- the reference's slice return -- or the argmax only), on
    # the same decode path, continuing after the generated tokens. Wall clock
    # per call.
    # Then the same with resident single steps (vvli_gpu_set_resident: the
    # launch stays and takes the next call's token through pinned memory).
    ft = {}
    n_ft = 32
    resident = persistent
    if args.prompt + args.steps + (6 if resident else 3) * n_ft <= args.ctx:
        pos = args.prompt + args.steps
        tok = int(tokens[-1])
        for suffix in ("", "_resident") if resident else ("",):
            runner.set_resident(2000 if suffix else 0)
            for kind in ("logits", "view", "argmax"):
                torch.cuda.synchronize()
                t1 = time.perf_counter()
                for _ in range(n_ft):
                    if kind == "logits":
                        tok = int(np.argmax(runner.forward_token(tok, pos)))
                    elif kind == "view":
                        tok = int(np.argmax(runner.forward_token_view(tok, pos)))
                    else:
                        tok = runner.forward_token_argmax(tok, pos)
                    pos += 1
                ft[f"us_per_call_{kind}{suffix}"] = round((time.perf_counter() - t1) / n_ft * 1e6, 1)
        runner.set_resident(0)
        ft["calls"] = n_ft
        print(f"[bench] forward_token: {ft['us_per_call_logits']} us/call with logits into the caller's buffer, "
              f"{ft['us_per_call_view']} as the pinned view, {ft['us_per_call_argmax']} argmax only",
              file=sys.stderr, flush=True)
        if resident:
            print(f"[bench] forward_token, resident steps: {ft['us_per_call_logits_resident']} / "
                  f"{ft['us_per_call_view_resident']} / {ft['us_per_call_argmax_resident']} us/call",
                  file=sys.stderr, flush=True)

    # GEMV half of the metric: the isolated op at M = 1 on the five projection
    # shapes of the model (cold weights), HBM GB/s per shape.
    gemv_rows = [] if args.no_gemv_sweep else gemv_sweep(LINEAR_SHAPES, [1], log=False)
    gemv = {f"{r['N']}x{r['K']}": {"us": r["us"], "gbs": r["gbs"], "frac": r["frac"],
                                   "us_host_loop": r["us_host_loop"]} for r in gemv_rows}
    if gemv_rows:
        agg = (sum(2 * r["N"] * r["K"] + 4 * r["K"] + 4 * r["N"] for r in gemv_rows) / sum(r["us"] for r in gemv_rows)
               / 1e3)
        gemv["all_shapes"] = {"gbs": round(agg, 1), "frac": round(agg / HBM_PEAK_GBS, 4),
                              "timing": "per shape: HIP graph of back-to-back calls over >= 1 GiB of weight copies, median of 5 replays"}
        print("[bench] gemv M=1: " + ", ".join(f"{k} {v['gbs']:.0f}GB/s" for k, v in gemv.items()), file=sys.stderr,
              flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cb = cpu_baseline(cfg, blob, prompt, args.cpu_budget, 512, inv_freq)
        # Parity spot check: the GPU's greedy continuation of the same prompt.
        runner.kv_clear()
        g_tokens, _ = runner.generate_greedy_measured(prompt, len(cb["tokens"]), batched_prefill=batched)
        same = bool(np.array_equal(g_tokens, np.array(cb["tokens"], dtype=np.uint32)))
        n_cpu = len(cb["tokens"])
        cpu = {"value": round(n_cpu / cb["seconds"], 3), "unit": "tok/s", "cores": cb["threads"],
               "kind": "port", "cpu_model": cpu_model(),
               "sample": f"oracle (C restatement of the reference CPU path, {cb['threads']} threads, 16-lane f32 "
                         f"accumulators, per-call thread fan-out as linearInto) greedy decode of {n_cpu} tokens at "
                         f"positions {len(prompt)}-{len(prompt) + n_cpu - 1} after the same {len(prompt)}-token "
                         f"prompt (run untimed through the oracle's prompt pass), same weights; "
                         f"GPU tokens identical: {same}"}
        print(f"[bench] cpu baseline {cpu['value']} tok/s on {cb['threads']} threads ({cpu['cpu_model']}); "
              f"tokens identical: {same}", file=sys.stderr, flush=True)

    line = {
        "metric": "decode tok/s @bs1 + GEMV HBM GB/s (% of peak), Llama-3.2-1B bf16",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(decode_s * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{args.model} bf16 greedy decode, bs1", "prompt_tokens": args.prompt,
                   "decode_tokens": args.steps, "ctx": args.ctx, "kv_cache": "f32", "prefill": args.prefill,
                   "weights": source,
                   "rope": ("llama3 scaling (factor 32, low/high freq factors 1/4, original ctx 8192)"
                            if inv_freq is not None else f"theta {cfg.rope_theta:g}"),
                   "parallelism": "none (1 GPU)"},
        "prefill_tok_s": round(prefill_tok_s, 2),
        "step_roofline": {"bytes_per_token_avg": step_bytes // args.steps, "achieved": round(step_gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "kernels": {k: {"avg_us": round(v["avg_us"], 2), "gbs": round(v["gbs"], 1)} for k, v in kernels.items()},
        "gemv_m1": gemv or None,
        "forward_token": ft or None,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    runner.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())

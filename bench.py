#!/usr/bin/env python3
"""bench.py - decode tok/s at batch 1 and achieved HBM GB/s on the 35B-shaped
Q4_K_M qwen35moe model (the C3 configuration), one MI355X.

Workload: hidden 2048, 40 layers (30 gated delta-net + 10 GQA), 256 experts
top-8 with FFN 512 + shared expert 512, vocab 248320; every projection Q4_K
except attn_v / ffn_down_exps / ffn_down_shexp in Q6_K; N(0,0.02) random-init
weights synthesised in HBM with the repository generator's value streams; a
4096-token random prompt through the layer-major prefill (the reference's
default chunked delta scan) fills the Q8 KV cache; then greedy decode. A "step" is one token through the whole stack (40 layers +
lm_head + argmax), everything resident in HBM, the next token chosen on the
device.

Prints ONE JSON line (driver contract) with the roofline of the dominant
kernel (per-launch HIP-event timing of one eager step) and the CPU baseline
(the oracle port on a bounded sample on this host's cores). Also reported:
the prompt rate (`prefill_tok_s`; `prefill_wy_tok_s` with the delta-net
chunks on the matrix cores, ORNITH_HIP_DELTA_MFMA=1) and, with `--batch N`, `batch_decode`: N
sessions with their own prompts stepped together (Model.batch_step; null by
default, and null with the engine's refusal logged when the contexts are past
the exact attention walk, where the batch step is switched off).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import ornithology_amd as oa  # noqa: E402

METRIC = "decode tok/s @batch1 + achieved HBM GB/s (% of roofline), 35B-shaped Q4_K_M"
HBM_PEAK_GBS = 8000.0

C3 = dict(hidden=2048, n_layers=40, vocab=248320, full_interval=4, nh=16, nkv=2, hd=256,
          nk=16, nv=32, dhead=128, conv_k=4, ne=256, top_k=8, moe_inter=512, shared_inter=512,
          t_default=oa.Q4_K, t_attn_v=oa.Q6_K, t_ffn_down=oa.Q6_K, t_output=oa.Q4_K, t_embd=oa.Q4_K,
          seed=0, sigma=0.02)

# 397B-shaped MoE sized to one GPU: routed experts IQ2_XXS, the rest Q4_K
C4 = dict(hidden=4096, n_layers=60, vocab=248320, full_interval=4, nh=32, nkv=2, hd=256,
          nk=16, nv=64, dhead=128, conv_k=4, ne=512, top_k=10, moe_inter=1024, shared_inter=1024,
          t_default=oa.Q4_K, t_attn_v=oa.Q4_K, t_ffn_down=oa.Q4_K, t_output=oa.Q4_K, t_embd=oa.Q4_K,
          t_exps=oa.IQ2_XXS, seed=0, sigma=0.02)
# C2 matvec microbench: [in x out] shapes and weight types
C2_SHAPES = [(2048, 248320), (2048, 4096), (512, 2048)]
C2_TYPES = [oa.Q8_0, oa.Q4_K, oa.Q6_K, oa.IQ2_XXS]
C2_COLD_BYTES = 1 << 30          # distinct weight copies per cold measurement (> 256 MB of caches)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def tensor_names(cfg: dict) -> list[str]:
    names = ["token_embd.weight", "output_norm.weight", "output.weight"]
    for l in range(cfg["n_layers"]):
        b = f"blk.{l}."
        names += [b + "attn_norm.weight", b + "post_attention_norm.weight"]
        if l % cfg["full_interval"] == cfg["full_interval"] - 1:
            names += [b + s for s in ("attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_q_norm.weight",
                                      "attn_k_norm.weight", "attn_output.weight")]
        else:
            names += [b + s for s in ("attn_qkv.weight", "ssm_conv1d.weight", "ssm_a", "ssm_dt.bias",
                                      "ssm_norm.weight", "ssm_alpha.weight", "ssm_beta.weight",
                                      "attn_gate.weight", "ssm_out.weight")]
        names += [b + s for s in ("ffn_gate_inp.weight", "ffn_gate_exps.weight", "ffn_up_exps.weight",
                                  "ffn_down_exps.weight", "ffn_gate_shexp.weight", "ffn_up_shexp.weight",
                                  "ffn_down_shexp.weight", "ffn_gate_inp_shexp.weight")]
    return names


def bytes_per_token(model: oa.Model, cfg: dict, ctx_len: float) -> dict:
    """Algorithmic HBM bytes of one decode step at context ctx_len: weights
    actually read (every non-expert tensor, top-k experts of each stack, one
    embedding row) + Q8 KV read/write + delta state and conv window r+w."""
    a = model.arch
    w = 0.0
    for n in tensor_names(cfg):
        info = model.tensor_info(n)
        if info is None:
            continue
        if n == "token_embd.weight":
            w += info["nbytes"] / a["vocab"]
        elif "_exps." in n:
            w += info["nbytes"] * a["top_k"] / a["ne"]
        else:
            w += info["nbytes"]
    n_full = sum(1 for l in range(a["n_layers"]) if l % a["full_interval"] == a["full_interval"] - 1)
    n_lin = a["n_layers"] - n_full
    kv_pos = 2 * a["nkv"] * (a["hd"] + 4)               # K and V codes + scales of one position
    kv = n_full * kv_pos * (ctx_len + 1)                 # read all cached positions + write one
    cc = 2 * a["nk"] * a["dk"] + a["nv"] * a["dv"]
    state = n_lin * (2 * 4 * a["nv"] * a["dk"] * a["dv"] + 2 * 4 * (a["conv_k"] - 1) * cc)
    return dict(weights=w, kv=kv, state=state, total=w + kv + state)


TRAFFIC_COPY_BYTES = 512 << 20
TRAFFIC_REPS = 2
TRAFFIC_PROMPT = 1


def traffic_probe(kind: str) -> int:
    """Under rocprofv3 --pmc: a device-to-device copy of TRAFFIC_COPY_BYTES
    (the calibration kernel), then one token step and TRAFFIC_REPS
    back-to-back replays of one decode step's `kind` launches on the C3 model
    (so the kernel's dispatches are TRAFFIC_PROMPT + 1 + TRAFFIC_REPS equal
    passes)."""
    import torch
    a = torch.empty(TRAFFIC_COPY_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    ctx = oa.Context(0)
    model = ctx.synth(**C3)
    sess = model.session(64)
    for i in range(TRAFFIC_PROMPT):
        sess.step(i * 7919 % C3["vocab"])
    us, bpl, nps = sess.time_kind(kind, reps=TRAFFIC_REPS)
    print(json.dumps({"kind": kind, "launches_per_step": nps, "reps": TRAFFIC_REPS, "us_per_launch": us,
                      "bytes_per_launch": bpl, "copy_bytes": TRAFFIC_COPY_BYTES}), flush=True)
    sess.free()
    model.free()
    ctx.close()
    return 0


def _counter_rows(path: str, counter: str):
    import csv
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


def traffic_summarize(kind: str, fetch_csv: str, write_csv: str) -> int:
    """FETCH_SIZE / WRITE_SIZE are KiB per dispatch. Each is scaled by what it
    reads for the calibration copy (a copy of N bytes reads and writes N), and
    the last TRAFFIC_REPS x launches_per_step dispatches of the kernel are
    averaged (the replay of --traffic-probe)."""
    sym = KERNEL_SYMBOL.get(kind, kind)
    out = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _counter_rows(path, counter)
        copy = [v for _, n, v in rows if "copy" in n.lower() or "elementwise" in n.lower()]
        # plain and templated kernel names ("void oh_k_delta16<128, 4>(...)")
        kern = [v for _, n, v in rows if n.split("(")[0].split("<")[0].split()[-1] == sym]
        if not copy or not kern:
            print(f"traffic: no {counter} rows for the copy or {sym}", file=sys.stderr)
            return 1
        factor = max(copy) * 1024.0 / TRAFFIC_COPY_BYTES
        out[counter] = dict(copy_kib=max(copy), factor=factor, dispatches=len(kern), kern_kib=kern)
    n = min(out["FETCH_SIZE"]["dispatches"], out["WRITE_SIZE"]["dispatches"])
    # the probe makes TRAFFIC_PROMPT token steps, one warm-up pass and
    # TRAFFIC_REPS timed passes of the same launches; keep the timed ones
    take = n * TRAFFIC_REPS // (TRAFFIC_PROMPT + 1 + TRAFFIC_REPS)
    tf = ROOT / "profiles" / "traffic.json"
    prev = json.loads(tf.read_text()) if tf.exists() else {}
    fetch = out["FETCH_SIZE"]["kern_kib"][-take:]
    write = out["WRITE_SIZE"]["kern_kib"][-take:]
    fb = sum(fetch) / len(fetch) * 1024.0 / out["FETCH_SIZE"]["factor"]
    wb = sum(write) / len(write) * 1024.0 / out["WRITE_SIZE"]["factor"]
    prev[kind] = {"bytes_per_launch": round(fb + wb), "fetch_bytes_per_launch": round(fb),
                  "write_bytes_per_launch": round(wb), "dispatches_averaged": len(fetch),
                  "fetch_copy_factor": round(out["FETCH_SIZE"]["factor"], 4),
                  "write_copy_factor": round(out["WRITE_SIZE"]["factor"], 4)}
    tf.write_text(json.dumps(prev, indent=1) + "\n")
    print(json.dumps(prev[kind]))
    return 0


def traffic_per_launch(kind: str):
    """HBM bytes per launch of `kind` measured with rocprofv3 FETCH_SIZE +
    WRITE_SIZE counter passes (calibrated on a device copy of known size),
    from profiles/traffic.json when that measurement exists, else None."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(kind, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def profile_kernels(sess: oa.Session, reps: int) -> dict:
    agg: dict[str, list[float]] = {}
    for _ in range(reps):
        for kind, byts, ms in sess.profile_step():
            e = agg.setdefault(kind, [0, 0.0, 0.0])
            e[0] += 1
            e[1] += byts
            e[2] += ms
    return {k: dict(launches=v[0] / reps, bytes=v[1] / reps, ms=v[2] / reps) for k, v in agg.items()}


def cpu_host() -> dict:
    """This host's CPUs as the CPU baseline uses them: nproc, the CPUs this
    process may run on, the CPU model, the NUMA nodes, and the per-GPU CPU
    share the box grants (OMP_NUM_THREADS there)."""
    allowed = sorted(os.sched_getaffinity(0))
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    nodes = {}
    for d in sorted(Path("/sys/devices/system/node").glob("node[0-9]*")):
        cpus = set()
        try:
            for part in (d / "cpulist").read_text().strip().split(","):
                if part:
                    a, _, b = part.partition("-")
                    cpus.update(range(int(a), int(b or a) + 1))
        except OSError:
            continue
        nodes[int(d.name[4:])] = cpus
    share = os.environ.get("OMP_NUM_THREADS")
    return {"nproc": os.cpu_count(), "allowed": allowed, "model": model, "nodes": nodes,
            "share": int(share) if share and share.isdigit() else None}


def cpu_pin(host: dict) -> tuple:
    """Pin this process to the NUMA node holding most of its allowed CPUs (in
    process, no re-exec); threads = min(that node's allowed CPUs, 64) as the
    reference sizes its pool (src/ornith_rforward.c:811-812), capped by the
    box's per-GPU CPU share. Returns (node, cpus, threads, previous mask)."""
    prev = set(host["allowed"])
    node, cpus = None, prev
    if host["nodes"]:
        node = max(host["nodes"], key=lambda k: len(host["nodes"][k] & prev))
        cpus = host["nodes"][node] & prev or prev
    os.sched_setaffinity(0, cpus)
    threads = min(len(cpus), 64)
    if host["share"]:
        threads = min(threads, host["share"])
    return node, sorted(cpus), threads, prev


def cpu_baseline(model: oa.Model, cfg: dict, ctx_len: int, reps: int = 3, steps: int = 16) -> dict:
    """Oracle port (the C restatement of the reference path, same per-matvec
    thread fan-out) on this host, pinned to one NUMA node: a 4-layer slice
    (3 delta-net + 1 GQA) of the same weights with the full 248320-row
    lm_head, written to a GGUF; the session moved to ctx_len positions with
    a seeded Q8 KV cache (orc_session_seed_context: an oracle prefill of
    4096 tokens takes minutes), then `reps` repetitions of `steps` greedy
    decode steps and of the lm_head matvec alone, best and mean as `ornith
    bench` reports them (src/ornith_bench.c:108-146). Token time =
    lm_head + n_layers/4 x (slice step - lm_head)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import clibs
    L = clibs.oracle()
    host = cpu_host()
    node, cpus, threads, prev = cpu_pin(host)
    try:
        with tempfile.TemporaryDirectory() as td:
            path = str(Path(td) / "slice.gguf")
            log("cpu baseline: writing the 4-layer slice GGUF")
            clibs.write_model_gguf(model, cfg, path, n_layers=4)
            log(f"cpu baseline: slice written; oracle port on {threads} threads, NUMA node {node} "
                f"({len(cpus)} CPUs), context {ctx_len}")
            m = C.c_void_p()
            assert L.orc_model_load(path.encode(), C.byref(m)) == 0, L.orc_last_error()
            L.orc_model_set_threads(m, threads)
            s = L.orc_session_new(m, ctx_len + reps * steps + 8, 1)
            assert L.orc_session_seed_context(s, ctx_len, 1) == 0
            x = np.ones(cfg["hidden"], np.float32)
            y = np.zeros(cfg["vocab"], np.float32)
            head = model.tensor_info("output.weight")
            hw = model.tensor("output.weight").download(head["nbytes"])
            t_head, t_step = [], []
            tok = 7
            for _ in range(reps):
                t0 = time.perf_counter()
                L.orc_matvec(head["type"], C.c_void_p(hw.ctypes.data), cfg["hidden"], cfg["vocab"],
                             clibs.f32p(x), clibs.f32p(y), 0, threads)
                t_head.append(time.perf_counter() - t0)
                t0 = time.perf_counter()
                for _ in range(steps):
                    L.orc_session_step(s, tok)
                    tok = int(np.argmax(np.ctypeslib.as_array(L.orc_session_logits(s), (cfg["vocab"],))))
                t_step.append((time.perf_counter() - t0) / steps)
            L.orc_session_free(s)
            L.orc_model_free(m)
    finally:
        os.sched_setaffinity(0, prev)

    def tok_time(h, st):
        return h + (cfg["n_layers"] / 4) * max(st - h, 0.0)

    best = tok_time(min(t_head), min(t_step))
    mean = tok_time(sum(t_head) / reps, sum(t_step) / reps)
    nodes = {str(k): len(v) for k, v in host["nodes"].items()}
    return dict(value=round(1.0 / mean, 4), unit="tok/s", cores=threads, kind="port",
                best=round(1.0 / best, 4), mean=round(1.0 / mean, 4), reps=reps,
                host={"nproc": host["nproc"], "allowed_cpus": len(host["allowed"]), "cpu_model": host["model"],
                      "numa_nodes": nodes, "pinned_node": node, "pinned_cpus": len(cpus),
                      "gpu_cpu_share": host["share"]},
                sample=f"oracle port, 4-layer slice (3 DN + 1 GQA) of the same weights + full lm_head at "
                       f"{ctx_len} positions (seeded Q8 KV): {reps} reps x {steps} greedy steps "
                       f"(best {min(t_step) * 1e3:.1f} / mean {sum(t_step) / reps * 1e3:.1f} ms per step) and "
                       f"{reps} lm_head matvecs (best {min(t_head) * 1e3:.1f} ms); token time = head + "
                       f"{cfg['n_layers'] // 4} x (step - head) = {mean * 1e3:.1f} ms mean, {best * 1e3:.1f} ms "
                       f"best; {threads} threads pinned to NUMA node {node}")


def batch_decode(model: oa.Model, n: int, ctx_len: int, steps: int) -> dict:
    """n sessions, each with its own ctx_len-token random prompt, stepped
    together by Model.batch_step (one token per session per step, greedy);
    wall clock around `steps` steps after 3 warm-up steps."""
    sess = []
    rng = np.random.default_rng(1)
    for _ in range(n):
        s = model.session(ctx_len + steps + 8)
        s.eval(rng.integers(0, model.arch["vocab"], ctx_len, dtype=np.int64).astype(np.int32))
        sess.append(s)
    toks = np.array([int(np.argmax(s.logits())) for s in sess], np.int32)
    for _ in range(3):
        toks = model.batch_step(sess, toks)
    t0 = time.perf_counter()
    for _ in range(steps):
        toks = model.batch_step(sess, toks)
    el = time.perf_counter() - t0
    for s in sess:
        s.free()
    return {"sessions": n, "context_tokens": ctx_len, "steps": steps, "ms_per_step": round(el / steps * 1e3, 3),
            "tok_s": round(n * steps / el, 1)}


# profile kind -> kernel symbol (as rocprofv3 names it)
KERNEL_SYMBOL = {"matvec": "oh_k_mv_q4k", "matvec_q6k": "oh_k_mv_q6k", "matvec_q80": "oh_k_mv_q80",
                 "matvec_mixed": "oh_k_mv_mixed", "matvec_q4q6": "oh_k_mv_q4k6k", "moe_down": "oh_k_mv_down_narrow",
                 "delta_step": "oh_k_delta16", "delta_mv": "oh_k_delta_mv", "attn_main": "oh_k_attn_main",
                 "attn_combine": "oh_k_attn_combine", "attn_prep": "oh_k_attn_prep", "attn_scores": "oh_k_attn_scores",
                 "attn_walk": "oh_k_attn_walk",
                 "step_body": "oh_k_step", "step_head": "oh_k_step"}


def c2_bench(args) -> int:
    """C2: the quantized matvec over N(0, 0.02) weights encoded on the device
    (seeded), per type and [in x out] shape. Cold: launches go round-robin over
    distinct copies of the weights totalling >= 1 GiB (more than L2 + MALL),
    replayed as one HIP graph; hot: the same tensor every launch (also one
    graph). CPU: the
    oracle port's qdot / f32-fallback matvec on this host's cores."""
    sys.path.insert(0, str(ROOT / "tests"))
    import clibs
    L = clibs.oracle()
    host = cpu_host()
    node, cpus, ncores, prev = cpu_pin(host)
    log(f"C2 CPU leg: oracle port on {ncores} threads, NUMA node {node} ({len(cpus)} CPUs), {host['model']}")
    ctx = oa.Context(0)
    rows = []
    for (n, out) in C2_SHAPES:
        w = (np.random.default_rng(hash((n, out)) & 0xffff).standard_normal(n * out, dtype=np.float32)
             * np.float32(0.02))
        x = np.random.default_rng(1).standard_normal(n, dtype=np.float32)
        for t in C2_TYPES:
            name = clibs.TYPE_NAMES[t]
            enc = ctx.quantize(t, w)
            ncopy = max(2, min(512, -(-C2_COLD_BYTES // enc.nbytes)))
            ts = [ctx.upload(f"c2.{name}.{k}", t, enc, (n, out)) for k in range(ncopy)]
            iters = max(2 * ncopy, 64)
            cold = ctx.time_matvec_set(ts, iters)
            hot = ctx.time_matvec_set(ts[:1], 64)
            for tt in ts:
                tt.free()
            # CPU: one matvec of the same weights and activation
            y = np.zeros(out, np.float32)
            reps, t0 = 0, time.perf_counter()
            while reps < 1 or time.perf_counter() - t0 < args.cpu_seconds / 12:
                L.orc_matvec(t, clibs.bp(enc), n, out, clibs.f32p(x), clibs.f32p(y), 0, ncores)
                reps += 1
            cpu_ms = (time.perf_counter() - t0) / reps * 1e3
            r = {"type": name, "in": n, "out": out, "weight_bytes": int(enc.nbytes), "copies": ncopy,
                 "cold_us": round(cold * 1e3, 3), "cold_gbs": round(enc.nbytes / (cold * 1e-3) / 1e9, 1),
                 "hot_us": round(hot * 1e3, 3), "hot_gbs": round(enc.nbytes / (hot * 1e-3) / 1e9, 1),
                 "cpu_ms": round(cpu_ms, 3), "cpu_threads": ncores}
            log(f"C2 {name:8s} [{n} x {out}] {enc.nbytes / 1e6:8.2f} MB: cold {r['cold_us']:9.2f} us "
                f"({r['cold_gbs']:7.1f} GB/s), hot {r['hot_us']:9.2f} us ({r['hot_gbs']:7.1f} GB/s), "
                f"cpu {cpu_ms:9.3f} ms")
            rows.append(r)
        del w
    os.sched_setaffinity(0, prev)
    big = [r for r in rows if r["out"] == C2_SHAPES[0][1]]
    best = max(big, key=lambda r: r["cold_gbs"])
    print(json.dumps({"metric": "C2 quantized matvec, cold HBM GB/s of the weight stream", "value": best["cold_gbs"],
                      "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "data": "synthetic",
                      "config": {"workload": "ornith_qdot matvec microbench (C2)", "best": best["type"]},
                      "roofline": {"bound": "hbm", "achieved": best["cold_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                   "frac": round(best["cold_gbs"] / HBM_PEAK_GBS, 4)},
                      "rows": rows}), flush=True)
    ctx.close()
    return 0


def c5_bench(args) -> int:
    """C5: the C3 weights, a 32768-token random prompt through the chunked
    layer-major prefill (ORNITH_HIP_PREFILL_CHUNK tokens per chunk, 4096 by
    default), then greedy decode at batch 1 and
    at batch 8 (eight independent seeded prompts of the same length)."""
    ctx = oa.Context(0)
    model = ctx.synth(**C3)
    ctx.sync()
    T = args.ctx
    steps = args.steps
    sess = model.session(T + steps + 16)
    prompt = np.random.default_rng(0).integers(0, C3["vocab"], T, dtype=np.int64).astype(np.int32)
    t0 = time.perf_counter()
    sess.eval(prompt)
    t_pf = time.perf_counter() - t0
    log(f"C5 prompt of {T} tokens: {t_pf:.2f} s ({T / t_pf:.0f} tok/s)")
    ms = sess.time_decode(steps)
    log(f"C5 batch 1: {steps} steps after {T} tokens: {ms / steps:.3f} ms/step -> {steps / (ms / 1e3):.1f} tok/s")
    bpt = bytes_per_token(model, C3, T + steps / 2)
    sess.free()
    bt = None
    if args.batch > 0:
        try:
            bt = batch_decode(model, args.batch, T, args.batch_steps)
            log(f"C5 batch {args.batch}: {bt['ms_per_step']:.2f} ms/step -> {bt['tok_s']:.1f} tok/s")
        except oa.HipError as e:
            log(f"C5 batch decode skipped: {e}")
    tok_s = steps / (ms / 1e3)
    print(json.dumps({"metric": "C5 long-context decode tok/s after a chunked 32K prefill", "value": round(tok_s, 2),
                      "unit": "tok/s", "n_gpus": 1, "steps": steps, "ms_per_step": round(ms / steps, 4),
                      "higher_is_better": True, "data": "synthetic",
                      "config": {"workload": "35B-shaped decode after a 32768-token chunked prefill (C5)",
                                 "context_tokens": T, "prefill_chunk": int(os.environ.get("ORNITH_HIP_PREFILL_CHUNK", "4096")),
                                 "delta_scan": "wy-mfma" if os.environ.get("ORNITH_HIP_DELTA_MFMA") == "1" else "exact"},
                      "prefill_tok_s": round(T / t_pf, 1), "prefill_s": round(t_pf, 3),
                      "hbm_gbs_step": round(bpt["total"] * tok_s / 1e9, 1),
                      "bytes_per_token": {k: round(v) for k, v in bpt.items()}, "batch_decode": bt}), flush=True)
    model.free()
    ctx.close()
    return 0


def timeline(args) -> int:
    """C3 at the bench's context: where one decode step's time goes, stage by
    stage, printed as markdown. (1) The per-launch HIP-graph step: each
    launch of one eager step timed with HIP events (launch order, first delta
    and first full-attention layer shown, then the per-stage mean over all
    layers), and every kernel kind replayed back to back as in the roofline
    figure. (2) The persistent step kernel (ORNITH_HIP_STEP=1): each phase
    between grid barriers. (3) The persistent tagged-word decode kernel
    (ORNITH_HIP_DECODE=1): each operation's critical-path share (the last
    block's completion after the previous operation's) and, for the first
    matvec, delta and MoE-down operations, the median per-block sub-phases."""
    ctx = oa.Context(0)
    model = ctx.synth(**C3)
    sess = model.session(args.ctx + 64)
    sess.eval(np.random.default_rng(0).integers(0, C3["vocab"], args.ctx, dtype=np.int64).astype(np.int32))
    ms = sess.time_decode(32)
    print(f"# C3 decode stage timeline ({args.ctx}-token context)\n")
    print(f"HIP-graph step: {ms / 32:.3f} ms/token ({32 / (ms / 1e3):.1f} tok/s), 32 steps.\n")
    prof = sess.profile_step()
    names = {"matvec": "Q4_K matvec", "matvec_mixed": "mixed matvec", "matvec_q6k": "Q6_K matvec",
             "matvec_q4q6": "Q4_K/Q6_K matvec", "attn_scores": "attn scores (exact)",
             "attn_walk": "attn walk (exact)", "delta_mv": "delta step + Q4_K matvec"}
    full = C3["full_interval"]
    # launch sequence per layer: every C3 layer ends with its MoE down
    # projection (launch 0 is the embedding, the head's launches come last)
    per_layer, cur = [], []
    for rec in prof[1:]:
        cur.append(rec)
        if rec[0] == "moe_down":
            per_layer.append(cur)
            cur = []
    head = cur
    assert len(per_layer) == C3["n_layers"], (len(per_layer), C3["n_layers"])
    print("## 1. Per-launch step (eager, HIP events around every launch)\n")
    for l in (0, full - 1):
        kind = "full-attention" if l % full == full - 1 else "delta-net"
        print(f"Layer {l} ({kind}):\n\n| # | kernel | us | MB |\n|---|---|---|---|")
        for j, (k, b, t) in enumerate(per_layer[l]):
            print(f"| {j} | {names.get(k, k)} | {t * 1e3:.2f} | {b / 1e6:.2f} |")
        print()
    for kind, pick in (("delta-net", lambda l: l % full != full - 1), ("full-attention", lambda l: l % full == full - 1)):
        rows = [per_layer[l] for l in range(C3["n_layers"]) if pick(l)]
        n = len(rows[0])
        print(f"Mean over the {len(rows)} {kind} layers:\n\n| stage | kernel | us |\n|---|---|---|")
        tot = 0.0
        for j in range(n):
            us = float(np.mean([r[j][2] for r in rows])) * 1e3
            tot += us
            print(f"| {j} | {names.get(rows[0][j][0], rows[0][j][0])} | {us:.2f} |")
        print(f"| | layer total | {tot:.2f} |\n")
    print(f"Head: {', '.join(f'{k} {t * 1e3:.2f} us' for k, _, t in head)}; embedding {prof[0][2] * 1e3:.2f} us.\n")
    print("Kernel kinds replayed back to back (one step's launches of a kind, HIP graph):\n")
    print("| kind | launches/step | us/launch | MB/launch | GB/s |\n|---|---|---|---|---|")
    for k in sorted({k for k, _, _ in prof}):
        if sum(1 for kk, _, _ in prof if kk == k) < 2:
            continue                                   # a single launch: the replay times the graph launch
        try:
            us, bpl, nps = sess.time_kind(k, reps=3)
        except oa.HipError:
            continue
        print(f"| {k} | {nps} | {us:.2f} | {bpl / 1e6:.2f} | {bpl / (us * 1e-6) / 1e9:.1f} |")
    print()
    try:
        ph = sess.profile_phases()
        agg = {}
        for k, b, us in ph:
            e = agg.setdefault(k or "barrier tail", [0, 0.0])
            e[0] += 1
            e[1] += us
        total = sum(v[1] for v in agg.values())
        print("## 2. Persistent step kernel (phases between grid barriers)\n")
        print(f"One body launch: {total:.1f} us over {len(ph)} phases.\n\n| kind | phases | us total | us/phase |\n"
              "|---|---|---|---|")
        for k, (n, us) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
            print(f"| {k} | {n} | {us:.1f} | {us / n:.2f} |")
        print()
    except oa.HipError as e:
        print(f"## 2. Persistent step kernel: unavailable ({e})\n")
    try:
        ops = sess.profile_decode()
        print("## 3. Persistent tagged-word decode kernel\n")
        crit = {}
        prev = 0.0
        for k, first, last in ops:
            e = crit.setdefault(k, [0, 0.0])
            e[0] += 1
            e[1] += last - prev
            prev = last
        print(f"One launch: {ops[-1][2]:.1f} us over {len(ops)} operations (critical path: each operation's "
              "last block done after the previous one's).\n\n| operation | count | us total | us/op |\n|---|---|---|---|")
        for k, (n, us) in sorted(crit.items(), key=lambda kv: -kv[1][1]):
            print(f"| {k} | {n} | {us:.1f} | {us / n:.2f} |")
        print("\nPer-block sub-phases (median over blocks, us): start -> inputs in LDS (the front wave's "
              "fetch) -> activation formed -> done (the delta operation stamps only its start and end).\n\n"
              "| op | kind | inputs | activation | dot + store | block total |\n|---|---|---|---|---|---|")
        want = {"matvec": None, "delta": None, "moe_down": None}
        for i, (k, _, _) in enumerate(ops):
            if k in want and want[k] is None:
                want[k] = i
        for k, i in want.items():
            if i is None:
                continue
            g = sess.profile_decode_op(i)
            tot = float(np.median(g[:, 5] - g[:, 0]))
            if np.all(g[:, 2] == 0):
                print(f"| {i} | {k} | | | | {tot:.2f} |")
                continue
            d = np.median(np.diff(g[:, [0, 2, 4, 5]], axis=1), axis=0)
            print(f"| {i} | {k} | {d[0]:.2f} | {d[1]:.2f} | {d[2]:.2f} | {tot:.2f} |")
        print()
    except oa.HipError as e:
        print(f"## 3. Persistent decode kernel: unavailable ({e})\n")
    sess.free()
    model.free()
    ctx.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", choices=("c3", "c2", "c4", "c5"), default="c3",
                    help="c3: the headline decode bench (default); c2: matvec microbench; c4: 397B-shaped "
                         "IQ2_XXS-expert decode; c5: 32K prefill + long-context decode at batch 1 and 8")
    ap.add_argument("--steps", type=int, default=None, help="decode steps (c3 256, c4 128, c5 512)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=None, help="prompt tokens before decode (c3 4096, c4 2048, c5 32768)")
    ap.add_argument("--profile-reps", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--batch", type=int, default=0,
                    help="sessions of the batch-decode figure (0: skip; the batch step refuses contexts past the "
                         "exact attention walk, so the figure is off by default)")
    ap.add_argument("--batch-steps", type=int, default=32)
    ap.add_argument("--timeline", action="store_true",
                    help="print where one C3 decode step's time goes, stage by stage (markdown), then exit")
    ap.add_argument("--traffic-probe", metavar="KIND", default=None,
                    help="run one device copy of known size and a replay of one step's KIND launches "
                         "(for rocprofv3 FETCH_SIZE / WRITE_SIZE passes), then exit")
    ap.add_argument("--traffic-summarize", nargs=3, metavar=("KIND", "FETCH_CSV", "WRITE_CSV"), default=None,
                    help="turn the two counter CSVs of --traffic-probe runs into profiles/traffic.json")
    args = ap.parse_args()
    if args.timeline:
        args.ctx = 4096 if args.ctx is None else args.ctx
        return timeline(args)
    if args.traffic_probe:
        return traffic_probe(args.traffic_probe)
    if args.traffic_summarize:
        return traffic_summarize(*args.traffic_summarize)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "multi-GPU sharding is a design, not a code path, in this build", file=sys.stderr)
        return 2
    dflt = {"c3": (4096, 256), "c4": (2048, 128), "c5": (32768, 512), "c2": (0, 0)}[args.config]
    args.ctx = dflt[0] if args.ctx is None else args.ctx
    args.steps = dflt[1] if args.steps is None else args.steps
    if args.config == "c2":
        return c2_bench(args)
    if args.config == "c5":
        return c5_bench(args)
    cfg = C3 if args.config == "c3" else C4
    metric = METRIC
    if args.config == "c4":
        metric = "decode tok/s @batch1 + achieved HBM GB/s (% of roofline), 397B-shaped, IQ2_XXS routed experts"
        args.batch = 0
        workload = ("397B-shaped qwen35moe decode sized to one GPU, batch 1, routed experts IQ2_XXS, the rest Q4_K, "
                    f"{args.ctx}-token Q8 KV context, greedy")
        dtype = "f32 (IQ2_XXS experts: the reference's f32 fallback) + int8 dot (Q8_K x Q4_K)"
    else:
        workload = ("35B-shaped qwen35moe decode, batch 1, Q4_K_M mix (Q6_K attn_v/ffn_down), "
                    f"{args.ctx}-token Q8 KV context, greedy")
        dtype = "int8 dot (Q8_K x Q4_K/Q6_K) + f32"

    if os.environ.get("ORNITH_HIP_NO_GRAPH") == "1" and args.batch > 0:
        log("ORNITH_HIP_NO_GRAPH=1: the batch-decode figure needs HIP graphs, skipped")
        args.batch = 0
    ctx = oa.Context(0)
    t0 = time.perf_counter()
    model = ctx.synth(**cfg)
    ctx.sync()
    t_synth = time.perf_counter() - t0
    log(f"synthesised {args.config} model in HBM: {model.nbytes / 1e9:.2f} GB in {t_synth:.1f} s")
    cap = args.ctx + args.warmup + args.steps + args.profile_reps + 8
    sess = model.session(cap)
    prompt = np.random.default_rng(0).integers(0, cfg["vocab"], args.ctx, dtype=np.int64).astype(np.int32)
    t0 = time.perf_counter()
    sess.eval(prompt)
    t_prefill = time.perf_counter() - t0
    log(f"prompt of {args.ctx} tokens through the layer-major prefill: {t_prefill:.2f} s "
        f"({args.ctx / t_prefill:.0f} tok/s)")
    # the same prompt with the delta-net chunks on the matrix cores (the WY
    # form, a tolerance path) in a session of its own
    t_prefill_wy = None
    if args.config == "c3" and os.environ.get("ORNITH_HIP_DELTA_MFMA") is None:
        os.environ["ORNITH_HIP_DELTA_MFMA"] = "1"
        try:
            sw = model.session(args.ctx + 8)
            ctx.sync()
            t0 = time.perf_counter()
            sw.eval(prompt)
            ctx.sync()
            t_prefill_wy = time.perf_counter() - t0
            sw.free()
        finally:
            del os.environ["ORNITH_HIP_DELTA_MFMA"]
        log(f"the same prompt with the matrix-core delta scan: {t_prefill_wy:.2f} s "
            f"({args.ctx / t_prefill_wy:.0f} tok/s)")

    if args.warmup:
        sess.time_decode(args.warmup)
    ctx.sync()
    w0 = time.perf_counter()
    ms = sess.time_decode(args.steps)
    ctx.sync()
    wall = time.perf_counter() - w0
    tok_s = args.steps / (ms / 1e3)
    log(f"timed {args.steps} decode steps: {ms:.2f} ms (events), {wall * 1e3:.2f} ms (wall) -> {tok_s:.1f} tok/s")

    ctx_mid = args.ctx + args.warmup + args.steps / 2
    bpt = bytes_per_token(model, cfg, ctx_mid)
    step_gbs = bpt["total"] * tok_s / 1e9

    # per-launch HIP events around every kernel of one eager step rank the
    # kernels; the dominant one is then timed by a back-to-back replay of its
    # launches (no per-launch event gaps), which is what the roofline uses
    prof = profile_kernels(sess, args.profile_reps)
    dom = max(prof, key=lambda k: prof[k]["ms"])
    for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"]):
        log(f"  {k:12s} {v['launches']:6.0f} launches  {v['ms']:8.3f} ms/step  {v['bytes'] / 1e6:9.1f} MB/step  "
            f"{v['bytes'] / max(v['ms'], 1e-9) / 1e6:8.1f} GB/s  (eager, per-launch events)")
    us, bpl, nps = sess.time_kind(dom, reps=args.profile_reps + 2)
    achieved = bpl / (us * 1e-6) / 1e9
    log(f"roofline kernel {KERNEL_SYMBOL.get(dom, dom)}: {nps} launches/step replayed back to back: "
        f"{us:.2f} us/launch, {bpl / 1e6:.2f} MB/launch -> {achieved:.1f} GB/s")

    batch = None
    if args.batch > 0:
        try:
            batch = batch_decode(model, args.batch, args.ctx, args.batch_steps)
            log(f"batch decode: {args.batch} sessions at {args.ctx} context: {batch['ms_per_step']:.2f} ms/step "
                f"-> {batch['tok_s']:.1f} tok/s")
        except oa.HipError as e:
            log(f"batch decode skipped: {e}")

    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(model, cfg, args.ctx)
            log(f"cpu baseline: {cpu['value']:.3f} tok/s mean, {cpu['best']:.3f} best, on {cpu['cores']} "
                f"threads ({cpu['host']})")
        except Exception as e:  # reported, never hides the GPU number
            log(f"cpu baseline failed: {e!r}")

    out = {
        "metric": metric, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dtype, "data": "synthetic",
        "config": {"workload": workload,
                   "context_tokens": args.ctx, "batch": 1, "weights_gb": round(model.nbytes / 1e9, 3),
                   "parallelism": "single GPU"},
        "hbm_gbs_step": round(step_gbs, 1), "roofline_frac_step": round(step_gbs / HBM_PEAK_GBS, 4),
        "bytes_per_token": {k: round(v) for k, v in bpt.items()},
        "roofline": {"bound": "hbm", "kernel": KERNEL_SYMBOL.get(dom, dom),
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_per_launch(dom),
                     "bytes_per_launch": round(bpl), "avg_launch_us": round(us, 3),
                     "launches_per_step": nps},
        "cpu_baseline": cpu,
        "prefill_tok_s": round(args.ctx / t_prefill, 1),
        "prefill_wy_tok_s": round(args.ctx / t_prefill_wy, 1) if t_prefill_wy else None,
        "batch_decode": batch,
    }
    print(json.dumps(out), flush=True)
    sess.free()
    model.free()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())

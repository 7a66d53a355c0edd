#!/usr/bin/env python3
"""Decode throughput of the inferox token loop on one MI355X.

Workload (one "step" = one greedy decode token at batch 1): the Llama-3-8B-shape
synthetic Q4_K_M model (dim 4096, 32 layers, 32/8 heads, ffn 14336, vocab
128256; Q4_K attn_q/k/o + ffn_gate/up + embedding, Q6_K attn_v/ffn_down/output),
a 2048-token KV context filled by a GPU prefill of 2048 seeded token ids, then
`--steps` greedy decode tokens timed end to end (weights and context resident
in HBM when timing starts).

Prints ONE JSON line (metric, value, roofline of the dominant kernel measured
with HIP events around back-to-back launches, with the same kernel timed by
event pairs around each launch of directly launched steps carried beside it;
cpu_baseline of the CPU oracle on a bounded sample).  `value` uses the f32 KV cache (the reference's; --kv f16
switches); `other_kv_cache` times the same decode with the other cache type,
reported apart from `value`.

Profiling aids: --no-graph launches each step's kernels directly instead of
replaying the captured step graph (for kernel tracers); --copy-probe only runs
a device-to-device copy of known size, the calibration for HBM byte counters;
--sampler T,K,P,SIGMA only runs 200 device draws (temperature T, top-k K,
top-p P) from 128256 seeded logits ~ N(0, SIGMA^2), for a kernel tracer;
--sampled-generate T,K,P times 256 tokens after a 512-id prompt, greedy and
drawn on the device, on the 8B model.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12  # B/s, MI355X HBM3E
CTX = 2048
METRIC = "decode tok/s, 8B Q4_K_M bs=1, 1×MI355X; % of HBM-BW roofline"
KCLASS = ["embed", "qkv_gemv", "attention", "attn_output_gemv", "ffn_gate_up_gemv", "ffn_down_gemv",
          "output_head_gemv", "finalize"]
# kernels of each class in the 8B / 70B decode step (the attention's merge runs
# in the O launch while a step attends at most 48 chunk records of 64 rows)
KERNEL_NAMES = {1: "k_gemv_mfma<EpiQkv, Q4_K, Q6_K>",
                2: "k_attn_decode<128, G> (+ k_attn_merge<128, G> past 48 chunks)",
                3: "k_gemv_ks_merge<Q4_K> (merge + O + residual; k_gemv_ks<Q4_K> past 48 chunks)",
                4: "k_gemv_mfma<EpiSwiglu, Q4_K>",
                5: "k_gemv_ks<Q6_K> (down + residual)", 6: "k_gemv_mfma<EpiLogits, Q6_K>"}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
COPY_PROBE_BYTES = 256 << 20


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--model", choices=["8b", "70b"], default="8b",
                    help="8b: Llama-3-8B shape, 2048-token context (the headline); 70b: Llama-3-70B shape, "
                         "8192-token context")
    ap.add_argument("--steps", type=int, default=None, help="decode tokens timed (8b: 256, 70b: 128)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--ctx", type=int, default=None, help="context tokens before the timed decode (8b: 2048, 70b: 8192)")
    ap.add_argument("--model-dir", default=os.environ.get("IFX_BENCH_DIR", os.path.join(tempfile.gettempdir(), "inferox_bench")))
    ap.add_argument("--cpu-steps", type=int, default=None,
                    help="oracle decode steps for cpu_baseline (0: skip; default 3 for 8b, 0 for 70b)")
    ap.add_argument("--no-micro", action="store_true", help="skip the GEMV microbench and the tiny-model run")
    ap.add_argument("--profile-steps", type=int, default=4)
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="direct launches instead of the step graph")
    ap.add_argument("--kv", choices=["f32", "f16"], default="f32",
                    help="KV cache element type: f32 (the reference's cache, the parity mode) or f16 (rounded rows)")
    ap.add_argument("--copy-probe", action="store_true", help="only a d2d copy of known size (counter calibration)")
    ap.add_argument("--sampler", default=None, metavar="T,K,P,SIGMA",
                    help="only 200 device draws from 128256 seeded logits (sampler kernel tracing)")
    ap.add_argument("--sampled-generate", default=None, metavar="T,K,P",
                    help="only 256 generated tokens after a 512-id prompt, greedy against sampled")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the batched prefill workload (512- and 2048-id prompts): tok/s, time to first token")
    ap.add_argument("--prefill-reps", type=int, default=3)
    ap.add_argument("--prefill-sizes", default="512,2048", help="prompt lengths of the prefill measurement")
    ap.add_argument("--lite", action="store_true",
                    help="decode, its profile and the CPU baseline only (no other-KV run, no prefill sizes)")
    ap.add_argument("--no-70b", action="store_true",
                    help="skip the 70B-shape run the default 8B line carries as model_70b")
    args = ap.parse_args()
    big = args.model == "70b"
    args.steps = args.steps if args.steps is not None else (128 if big else 256)
    args.ctx = args.ctx if args.ctx is not None else (8192 if big else CTX)
    args.cpu_steps = args.cpu_steps if args.cpu_steps is not None else (0 if big else 3)
    return args


def copy_probe():
    """8 launches of a plain copy kernel over COPY_PROBE_BYTES (an F32 tensor
    "dequantized" to f32: read N*4 bytes, write N*4 bytes).  Under a byte
    counter, the reading per launch against the known size is the counter's
    scale factor."""
    from inferox_amd import _native
    from inferox_amd._native import check
    L = _native.lib()
    n = COPY_PROBE_BYTES // 4
    host = np.zeros(n, np.float32)
    t = C.c_void_p()
    check(L.ifx_tensor_upload(0, host.ctypes.data_as(C.c_void_p), COPY_PROBE_BYTES, 1, n, C.byref(t)), "upload")
    out = C.c_void_p()
    check(L.ifx_malloc(C.byref(out), COPY_PROBE_BYTES), "malloc")
    for _ in range(8):
        check(L.ifx_tensor_dequant(t, out, None), "copy")
    check(L.ifx_stream_synchronize(None), "sync")
    L.ifx_free(out)
    L.ifx_tensor_free(t)
    print(json.dumps({"copy_probe_bytes": COPY_PROBE_BYTES, "launches": 8, "kernel": "k_dequant_dev"}), flush=True)


def sampler_probe(spec):
    """200 draws of ifx_sample_logits (temperature, top-k, top-p) from 128256
    logits ~ N(0, sigma^2) of a fixed seed: the sampler's launches (the logits'
    maximum, weights, plan and gather, select, finalize) 200 times, for a
    kernel tracer; the wall time includes the call's allocations and copies."""
    from inferox_amd import _native, synth
    T, K, P, sig = (float(v) for v in spec.split(","))
    z = (np.random.default_rng(5).standard_normal(synth.LLAMA3_8B.vocab) * sig).astype(np.float32)
    out = np.zeros(200, np.uint32)
    L = _native.lib()
    t0 = time.perf_counter()
    rc = L.ifx_sample_logits(z.ctypes.data_as(C.c_void_p), z.size, T, int(K), P, 9, out.size,
                             out.ctypes.data_as(C.c_void_p))
    wall = time.perf_counter() - t0
    if rc != 0:
        raise SystemExit(f"ifx_sample_logits: {(L.ifx_last_error() or b'').decode()}")
    print(json.dumps({"sampler": {"temperature": T, "top_k": int(K), "top_p": P, "sigma": sig},
                      "vocab": int(z.size), "draws": int(out.size), "wall_ms": round(wall * 1e3, 2),
                      "distinct_tokens": int(np.unique(out).size)}), flush=True)


def traffic_for(kclass):
    """HBM bytes per launch of a kernel class from the committed counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the factor
    measured on a copy of known size), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        k = t["kernels"][kclass]
        return int(k["fetch_kib"] * 1024 * t["fetch_factor"] + k["write_kib"] * 1024 * t["write_factor"])
    except (OSError, KeyError, ValueError, TypeError):
        return None


MFMA_PEAK_F16 = 2.5e15  # FLOP/s, MI355X dense fp16


def prefill_flops(spec, n):
    """Algorithmic FLOPs of a prefill of n ids: every linear layer on every row
    (2 per weight element), the output matrix on the last row only, and the
    causal attention (q.k and p.v over the n(n+1)/2 visible pairs per head)."""
    D, F, KV = spec.dim, spec.ffn, spec.kv_dim
    per_row = 2 * spec.n_layers * (2 * D * D + 2 * D * KV + 3 * D * F)
    attn = spec.n_layers * spec.n_heads * (n * (n + 1) // 2) * spec.head_dim * 4
    return n * per_row + 2 * spec.vocab * D + attn


def measure_other_kv(L, model, spec, kv_type, ctx, steps, warmup):
    """The same decode with the other KV cache type (reported apart from `value`):
    a fresh session, the same seeded context through the batched prefill, warmup,
    then `steps` greedy tokens timed."""
    from inferox_amd import synth
    from inferox_amd._native import check
    sess = C.c_void_p()
    check(L.ifx_session_create_kv(model, ctx + max(steps, warmup) + 8, kv_type, C.byref(sess)), "session_create_kv")
    out = np.zeros(max(steps, warmup, 1), np.uint32)
    check(L.ifx_decode_greedy(sess, 1, warmup, out.ctypes.data_as(C.c_void_p)), "warmup")
    check(L.ifx_session_clear(sess), "clear")
    ids = synth.token_ids(ctx, spec.vocab, seed=2048)
    check(L.ifx_prefill(sess, ids.ctypes.data_as(C.c_void_p), ids.size, None), "prefill")
    first = C.c_uint32()
    check(L.ifx_session_last_token(sess, C.byref(first)), "last_token")
    check(L.ifx_stream_synchronize(None), "sync")
    t0 = time.perf_counter()
    check(L.ifx_decode_greedy(sess, first.value, steps, out.ctypes.data_as(C.c_void_p)), "decode")
    wall = time.perf_counter() - t0
    L.ifx_session_destroy(sess)
    return {"kv_cache": "f16" if kv_type == 1 else "f32", "tok_s": round(steps / wall, 2),
            "ms_per_step": round(wall / steps * 1e3, 4), "first_tokens": [int(x) for x in out[:4]]}


def measure_sampled_generate(L, model, spec, cfg):
    """256 tokens generated after a 512-id prompt, greedy (ifx_generate)
    against drawn by the device sampler (ifx_generate_sampled: temperature,
    top-k, top-p, seed 7), alternated twice; the device-loop time of each call
    (ifx_session_last_elapsed_ms)."""
    from inferox_amd import synth
    from inferox_amd._native import check
    T, K, P = cfg.split(",")
    T, K, P = float(T), int(K), float(P)
    sess = C.c_void_p()
    check(L.ifx_session_create(model, 1024, C.byref(sess)), "session_create")
    ids = synth.token_ids(512, spec.vocab, seed=3)
    out = np.zeros(256, np.uint32)
    res = {"greedy": [], "sampled": []}
    check(L.ifx_session_set_sampler(sess, T, K, P, 7), "set_sampler")
    for mode in ("greedy", "sampled", "greedy", "sampled"):
        f = L.ifx_generate_sampled if mode == "sampled" else L.ifx_generate
        check(f(sess, ids.ctypes.data_as(C.c_void_p), ids.size, out.size, out.ctypes.data_as(C.c_void_p)), mode)
        ms = C.c_float()
        check(L.ifx_session_last_elapsed_ms(sess, C.byref(ms)), "elapsed")
        res[mode].append(round(out.size / ms.value * 1e3, 1))
    L.ifx_session_destroy(sess)
    return {"sampled_generate": {"temperature": T, "top_k": K, "top_p": P, "seed": 7},
            "workload": f"{spec.name}: 512-id prompt, 256 generated tokens, device loop",
            "greedy_tok_s": res["greedy"], "sampled_tok_s": res["sampled"]}


def measure_prefill(L, model, spec, sizes, reps):
    """Batched prefill of seeded prompts: best of `reps` runs each, wall time
    from the ids on the host to the first generated token id on the host."""
    from inferox_amd._native import check
    out = {}
    for n in sizes:
        sess = C.c_void_p()
        check(L.ifx_session_create(model, n + 8, C.byref(sess)), "session_create")
        ids = __import__("inferox_amd.synth", fromlist=["synth"]).token_ids(n, spec.vocab, seed=512 + n)
        first = C.c_uint32()
        best = None
        dev_ms = None
        for r in range(reps + 1):  # the first run allocates the workspace
            check(L.ifx_session_clear(sess), "clear")
            check(L.ifx_stream_synchronize(None), "sync")
            t0 = time.perf_counter()
            check(L.ifx_prefill(sess, ids.ctypes.data_as(C.c_void_p), n, None), "prefill")
            check(L.ifx_session_last_token(sess, C.byref(first)), "last_token")
            dt = time.perf_counter() - t0
            if r > 0 and (best is None or dt < best):
                best = dt
                ms = C.c_float()
                L.ifx_session_last_elapsed_ms(sess, C.byref(ms))
                dev_ms = ms.value
        L.ifx_session_destroy(sess)
        fl = prefill_flops(spec, n)
        out[f"p{n}"] = {"tokens": n, "tok_s": round(n / best, 1), "ttft_ms": round(best * 1e3, 2),
                        "device_ms": round(dev_ms, 2), "tflop": round(fl / 1e12, 3),
                        "mfma_frac": round(fl / (dev_ms * 1e-3) / MFMA_PEAK_F16, 4), "first_token": int(first.value)}
        log(f"prefill {n}: {out[f'p{n}']}")
    return out


def host_cpu():
    """The host the CPU baseline ran on: model name, cores visible to this
    process, and whether the AVX2 / FMA paths of matmul_t apply."""
    model, flags = None, set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model is None:
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count()
    return {"cpu_model": model, "nproc": avail, "os_cpu_count": os.cpu_count(), "avx2": "avx2" in flags,
            "fma": "fma" in flags, "avx512f": "avx512f" in flags}


# The GEMV microbench: four weight shapes, x ~ N(0, 1) f32, timed over copies
# of each matrix that together hold at least MICRO_BYTES (past the 256 MB
# memory-side cache), each call on the next copy.
MICRO_SHAPES = [("q4k_4096x4096", 12, 4096, 4096), ("q4k_14336x4096", 12, 14336, 4096),
                ("q4k_4096x14336", 12, 4096, 14336), ("q6k_128256x4096", 14, 128256, 4096)]
MICRO_BYTES = 512 << 20


def gemv_microbench(L, rounds=8):
    """Per shape: microseconds per call, algorithmic GB/s (weight bytes + f32 x
    and y) and the fraction of 8 TB/s, HIP events around `rounds` passes over
    the rotating copies on the library stream."""
    from inferox_amd import synth
    from inferox_amd._native import check
    from inferox_amd.synth import byte_size
    res = {}
    for name, t, rows, cols in MICRO_SHAPES:
        wb = byte_size(t, rows * cols)
        n_copies = max(2, -(-MICRO_BYTES // wb))
        raw = synth.random_blocks(t, rows * cols, seed=rows * 7 + cols)
        tens = []
        for _ in range(n_copies):
            h = C.c_void_p()
            check(L.ifx_tensor_upload(t, raw.ctypes.data_as(C.c_void_p), raw.size, rows, cols, C.byref(h)), "upload")
            tens.append(h)
        x = synth.normal_f32(cols, seed=cols)
        dx, dy = C.c_void_p(), C.c_void_p()
        check(L.ifx_malloc(C.byref(dx), cols * 4), "malloc")
        check(L.ifx_malloc(C.byref(dy), rows * 4), "malloc")
        check(L.ifx_memcpy_h2d(dx, x.ctypes.data_as(C.c_void_p), cols * 4), "h2d")
        for h in tens:  # warm: one pass
            check(L.ifx_gemv(h, dx, dy, None), "gemv")
        check(L.ifx_timer_start(None), "timer")
        for _ in range(rounds):
            for h in tens:
                check(L.ifx_gemv(h, dx, dy, None), "gemv")
        ms = C.c_float()
        check(L.ifx_timer_stop(None, C.byref(ms)), "timer")
        calls = rounds * n_copies
        us = ms.value * 1e3 / calls
        b = wb + 4 * (rows + cols)
        res[name] = {"rows": rows, "cols": cols, "type": "Q4_K" if t == 12 else "Q6_K", "bytes_per_call": b,
                     "copies": n_copies, "calls": calls, "us": round(us, 3), "GB_s": round(b / (us * 1e-6) / 1e9, 1),
                     "frac": round(b / (us * 1e-6) / HBM_PEAK, 4)}
        log(f"gemv {name}: {res[name]}")
        L.ifx_free(dx)
        L.ifx_free(dy)
        for h in tens:
            L.ifx_tensor_free(h)
    return res


def tiny_run(L, model_dir, cpu: bool):
    """The tiny Q8_0 workload end to end: a 16-token seeded prompt, then 128
    greedy tokens (ctx 256), through ifx_generate; tok/s of the generated
    tokens (prefill included, as the workload defines it), and the faithful
    CPU restatement on one thread over the same workload when `cpu`."""
    from inferox_amd import synth
    from inferox_amd._native import check
    path = os.path.join(model_dir, "tiny-seed1234.gguf")
    if not os.path.exists(path):
        synth.write_llama(path, synth.TINY, seed=1234)
    prompt = synth.token_ids(16, synth.TINY.vocab, seed=4321)
    model = C.c_void_p()
    check(L.ifx_model_open(path.encode(), C.byref(model)), "tiny open")
    sess = C.c_void_p()
    check(L.ifx_session_create(model, 256, C.byref(sess)), "tiny session")
    out = np.zeros(128, np.uint32)
    check(L.ifx_generate(sess, prompt.ctypes.data_as(C.c_void_p), 16, 128, out.ctypes.data_as(C.c_void_p)), "warm")
    best = None
    for _ in range(3):
        check(L.ifx_stream_synchronize(None), "sync")
        t0 = time.perf_counter()
        check(L.ifx_generate(sess, prompt.ctypes.data_as(C.c_void_p), 16, 128, out.ctypes.data_as(C.c_void_p)),
              "tiny generate")
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    L.ifx_session_destroy(sess)
    L.ifx_model_close(model)
    r = {"workload": "tiny Q8_0 (dim 288, 6 layers, vocab 32000): 16-token prompt + 128 greedy tokens, ctx 256",
         "tok_s": round(128 / best, 1), "ms_total": round(best * 1e3, 2), "first_tokens": [int(v) for v in out[:4]]}
    if cpu:
        from oracle import binding as orc
        orc.set_threads(1)
        m = orc.Model(path)
        kv = m.kv(256)
        t0 = time.perf_counter()
        rc, ref = m.generate(kv, prompt, 128, mode=orc.MODE_FAITHFUL)
        dt = time.perf_counter() - t0
        m.close()
        r["cpu_tok_s"] = round(128 / dt, 2)
        r["cpu_kind"] = "port (faithful restatement, 1 thread)"
        r["tokens_equal_cpu"] = bool(rc == 0 and ref.tolist() == out.tolist())
    log(f"tiny: {r}")
    return r


def bytes_per_token(spec, ctx_avg):
    """Stored weight bytes read per decode token (one embedding row, all layers,
    final norm, output) + KV at a canonical 2 B/element."""
    from inferox_amd.synth import byte_size
    total = 0
    for name, _, t, r, c in spec.shapes():
        if name == "token_embd.weight":
            total += byte_size(t, c)          # one row
        else:
            total += byte_size(t, r * c)
    kv = 2 * spec.n_layers * ctx_avg * spec.kv_dim * 2
    return total, kv


def cpu_baseline(model_path, kv_k, kv_v, ctx, token, n_steps):
    """The reference algorithm (faithful CPU restatement: per-step full dequant
    into fresh buffers, AVX2 matmul_t, scalar ops), 1 thread, n_steps decode
    steps from the same KV state the GPU decoded from."""
    from oracle import binding as orc
    orc.set_threads(1)
    m = orc.Model(model_path)
    kv = m.kv(ctx + n_steps + 1)
    assert kv.import_(kv_k, kv_v, ctx) == 0
    times, toks = [], []
    t = token
    for _ in range(n_steps):
        t0 = time.perf_counter()
        rc, logits = m.decode_step(kv, t, mode=orc.MODE_FAITHFUL)
        times.append(time.perf_counter() - t0)
        assert rc == 0
        t = orc.argmax(logits)[1]
        toks.append(t)
    m.close()
    med = float(np.median(times))
    return med, toks


def run_70b(args):
    """The 70B-shape workload (8192-token context from a GPU prefill, then 128
    greedy tokens, f32 KV, one faithful CPU step from the same state) in a
    child process of this script, when the scratch space holds its 45 GB
    model; its JSON line, or why it was skipped."""
    import shutil
    import subprocess
    from inferox_amd import synth
    spec = synth.LLAMA3_70B
    path = os.path.join(args.model_dir, f"{spec.name}-seed1234.gguf")
    have = os.path.exists(path) and os.path.getsize(path) >= spec.gguf_bytes()
    free = shutil.disk_usage(args.model_dir).free
    if not have and free < spec.gguf_bytes() + (4 << 30):
        return {"skipped": f"the 70B model needs {spec.gguf_bytes() / 1e9:.1f} GB of scratch space; "
                           f"{free / 1e9:.1f} GB free in {args.model_dir}"}
    cmd = [sys.executable, os.path.abspath(__file__), "--model", "70b", "--steps", "128", "--warmup", "8",
           "--cpu-steps", "1", "--no-micro", "--lite", "--model-dir", args.model_dir]
    log("70B-shape run: " + " ".join(cmd[1:]))
    try:
        r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=1200)
    except subprocess.TimeoutExpired:
        return {"skipped": "the 70B-shape run did not finish in 1200 s"}
    lines = [x for x in r.stdout.splitlines() if x.startswith("{")]
    if r.returncode != 0 or not lines:
        return {"skipped": f"the 70B-shape run failed (exit {r.returncode})"}
    d = json.loads(lines[-1])
    keep = ("metric", "value", "unit", "steps", "warmup", "ms_per_step", "dtype", "config", "roofline",
            "roofline_tok", "device_tok_s", "prefill_tok_s", "cpu_baseline", "kernels")
    return {k: d.get(k) for k in keep}


def main():
    args = parse()
    if args.no_graph:
        os.environ["IFX_NO_GRAPH"] = "1"  # read by the library at the first step
    if args.copy_probe:
        copy_probe()
        return
    if args.sampler:
        sampler_probe(args.sampler)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU: the token loop runs on a single MI355X; "
                          "multi-GPU sharding (heads and FFN columns split per GPU) is not built",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    from inferox_amd import _native, synth
    from inferox_amd._native import check
    L = _native.lib()

    spec = synth.LLAMA3_70B if args.model == "70b" else synth.LLAMA3_8B
    os.makedirs(args.model_dir, exist_ok=True)
    path = os.path.join(args.model_dir, f"{spec.name}-seed1234.gguf")
    if not os.path.exists(path) or os.path.getsize(path) < spec.gguf_bytes():
        log(f"writing synthetic {spec.name} ({spec.gguf_bytes() / 1e9:.2f} GB) to {path}")
        t0 = time.time()
        synth.write_llama(path, spec, seed=1234)
        log(f"  written in {time.time() - t0:.1f} s")

    name = C.create_string_buffer(128)
    ncu, hbm = C.c_int(), C.c_uint64()
    check(L.ifx_device_info(name, 128, C.byref(ncu), C.byref(hbm)), "device_info")
    log(f"device: {name.value.decode()} CUs={ncu.value} HBM={hbm.value / 2**30:.0f} GiB")

    t0 = time.time()
    model = C.c_void_p()
    check(L.ifx_model_open(path.encode(), C.byref(model)), "model_open")
    dev_b, gguf_b = C.c_uint64(), C.c_uint64()
    L.ifx_model_weight_bytes(model, C.byref(dev_b), C.byref(gguf_b))
    log(f"model uploaded in {time.time() - t0:.1f} s: {dev_b.value / 1e9:.3f} GB in HBM "
        f"({gguf_b.value / 1e9:.3f} GB stored)")

    if args.sampled_generate:
        print(json.dumps(measure_sampled_generate(L, model, spec, args.sampled_generate)), flush=True)
        return
    if args.prefill_only:
        sizes = [int(x) for x in args.prefill_sizes.split(",")]
        res = measure_prefill(L, model, spec, sizes, args.prefill_reps)
        L.ifx_model_close(model)
        print(json.dumps({"metric": f"prefill tok/s, {args.model.upper()} Q4_K_M, 1xMI355X", "unit": "tok/s",
                          "value": res[f"p{sizes[-1]}"]["tok_s"], "higher_is_better": True, "dtype": "f16x3 (f32 accumulate)",
                          "data": "synthetic", "config": {"workload": f"{spec.name}-shape Q4_K_M batched prefill of "
                                                                      "seeded 512- and 2048-id prompts"},
                          "prefill": res}), flush=True)
        return

    K, W = args.steps, args.warmup
    max_seq = args.ctx + max(K, W) + 2 * args.profile_steps + 8
    sess = C.c_void_p()
    check(L.ifx_session_create_kv(model, max_seq, 1 if args.kv == "f16" else 0, C.byref(sess)), "session_create")
    vocab = spec.vocab

    # warmup on an empty cache (graph capture, clocks), then the real context
    out = np.zeros(max(K, W, 1), np.uint32)
    check(L.ifx_decode_greedy(sess, 1, W, out.ctypes.data_as(C.c_void_p)), "warmup")
    check(L.ifx_session_clear(sess), "clear")
    ms = C.c_float()
    prefill_s = None
    if args.ctx > 0:
        ids = synth.token_ids(args.ctx, vocab, seed=2048)
        t0 = time.perf_counter()
        check(L.ifx_prefill(sess, ids.ctypes.data_as(C.c_void_p), ids.size, None), "prefill")
        prefill_s = time.perf_counter() - t0
        log(f"prefill of {args.ctx} tokens: {prefill_s:.2f} s ({args.ctx / prefill_s:.0f} tok/s)")
        # the first generated token = greedy pick of the last prefill row (Model::generate)
        first = C.c_uint32()
        check(L.ifx_session_last_token(sess, C.byref(first)), "last_token")
        start_tok = first.value
    else:  # --ctx 0: decode from an empty cache (short runs under counters)
        start_tok = 1
    kv_len = C.c_uint64()
    L.ifx_session_len(sess, C.byref(kv_len))
    assert kv_len.value == args.ctx
    # the context is exported for the CPU baseline before decoding further
    n_kv = spec.n_layers * args.ctx * spec.kv_dim
    do_cpu = args.cpu_steps > 0
    kv_k = np.zeros(n_kv if do_cpu else 1, np.float32)
    kv_v = np.zeros_like(kv_k)
    if do_cpu:
        check(L.ifx_kv_export(sess, kv_k.ctypes.data_as(C.c_void_p), kv_v.ctypes.data_as(C.c_void_p), args.ctx),
              "kv_export")

    # ---- timed region: K greedy decode steps, synchronized on both sides ----
    check(L.ifx_stream_synchronize(None), "sync")
    t0 = time.perf_counter()
    check(L.ifx_decode_greedy(sess, start_tok, K, out.ctypes.data_as(C.c_void_p)), "decode")
    wall = time.perf_counter() - t0
    L.ifx_session_last_elapsed_ms(sess, C.byref(ms))
    dev_s = ms.value / 1e3
    tok_s = K / wall
    log(f"decode {K} tokens: wall {wall * 1e3:.1f} ms ({tok_s:.1f} tok/s), device {dev_s * 1e3:.1f} ms "
        f"({K / dev_s:.1f} tok/s)")

    w_bytes, kv_bytes = bytes_per_token(spec, args.ctx + (K + 1) / 2)
    b_tok = w_bytes + kv_bytes
    frac_tok = tok_s * b_tok / HBM_PEAK

    # ---- dominant kernel: HIP events around each launch of directly launched
    # steps (step order: each kernel meets the cache state of a real step), and
    # around back-to-back launches of each class (reported beside it) ----
    roofline = None
    prof = {}
    if not args.no_profile:
        avg = (C.c_float * 8)()
        ordered = (C.c_float * 8)()
        launches = (C.c_uint64 * 8)()
        wbytes = (C.c_uint64 * 8)()
        check(L.ifx_session_profile_ordered(sess, int(out[K - 1]), args.profile_steps, ordered), "profile_ordered")
        check(L.ifx_session_profile(sess, int(out[K - 1]), args.profile_steps, avg, launches, wbytes), "profile")
        # avg: back-to-back launches of one class (kernel + the launch gap);
        # ordered (step order): an event pair around each launch, which adds the
        # events' own ~2 us per launch -- the two bracket the kernel's duration
        # inside the replayed step graph (rocprofv3 trace in profiles/)
        per_step = {KCLASS[k]: avg[k] * launches[k] for k in range(8)}
        dom = max(range(8), key=lambda k: avg[k] * launches[k])
        # algorithmic bytes of one launch of the dominant kernel: its weight bytes
        # + the f32 input vector (+ the f32 norm weight when the norm is fused)
        # (attention: the K/V rows it reads, reported by the library)
        extra = 0 if dom == 2 else ({1: 2, 4: 2, 6: 2}.get(dom, 1) * spec.dim * 4 if dom != 5 else spec.ffn * 4)
        alg = wbytes[dom] + extra
        achieved = alg / (avg[dom] * 1e-3)
        roofline = {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                    "traffic": traffic_for(KCLASS[dom]) if args.model == "8b" else None,
                    "traffic_source": ("rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch of this kernel at ctx 2048, "
                                       "scaled by a copy of known size (profiles/traffic.json; counters cannot run "
                                       "inside this process)") if args.model == "8b" else None,
                    "kernel": KERNEL_NAMES.get(dom, KCLASS[dom]), "kernel_class": KCLASS[dom],
                    "bytes_per_launch": int(alg), "avg_launch_us": round(avg[dom] * 1e3, 2),
                    "avg_launch_us_timing": "HIP events around 32 x profile_steps back-to-back launches on the "
                                            "session stream",
                    "avg_launch_us_step_order": round(ordered[dom] * 1e3, 2),
                    "frac_step_order": round(alg / (ordered[dom] * 1e-3) / HBM_PEAK, 4) if ordered[dom] else None}
        prof = {KCLASS[k]: {"avg_us": round(avg[k] * 1e3, 2), "step_order_us": round(ordered[k] * 1e3, 2),
                            "launches_per_step": int(launches[k]),
                            "weight_bytes": int(wbytes[k]),
                            "GB_s": round(wbytes[k] / (avg[k] * 1e-3) / 1e9, 1) if avg[k] > 0 and wbytes[k] else None}
                for k in range(8)}
        log("per-kernel (back-to-back; step order with its event pairs beside): " + json.dumps(prof))
        log(f"sum of kernel time per step: {sum(per_step.values()):.3f} ms vs {wall / K * 1e3:.3f} ms per step")

    cpu = None
    if do_cpu:
        log(f"cpu baseline: {args.cpu_steps} faithful oracle step(s) at ctx {args.ctx}, 1 thread ...")
        med, toks = cpu_baseline(path, kv_k, kv_v, args.ctx, start_tok, args.cpu_steps)
        cpu = {"value": round(1.0 / med, 4), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"{args.cpu_steps} decode step(s) of the same {args.model.upper()} model from the same {args.ctx}-row KV "
                         f"state, faithful CPU restatement (per-step full dequant, AVX2 matmul_t), median "
                         f"{med:.2f} s/step; greedy picks {toks} vs GPU {[int(v) for v in out[:len(toks)]]}",
               "host": host_cpu()}
        log(f"cpu: {med:.2f} s/step; first pick cpu={toks[0]} gpu={int(out[0])}")

    L.ifx_session_destroy(sess)
    other_kv = None
    if not args.no_profile and not args.lite:
        other_kv = measure_other_kv(L, model, spec, 0 if args.kv == "f16" else 1, args.ctx, K, W)
        log(f"decode with the {other_kv['kv_cache']} KV cache: {other_kv['tok_s']} tok/s")
    prefill = None if (args.no_profile or args.lite) else measure_prefill(
        L, model, spec, [int(x) for x in args.prefill_sizes.split(",")], 1)
    L.ifx_model_close(model)
    micro = tiny = None
    if not args.no_micro and args.model == "8b":
        micro = gemv_microbench(L)
        tiny = tiny_run(L, args.model_dir, cpu=do_cpu)
    model_70b = None
    if args.model == "8b" and not args.no_70b and not args.no_profile:
        model_70b = run_70b(args)

    line = {
        "metric": METRIC if args.model == "8b" else METRIC.replace("8B", "70B"), "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(wall / K * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{spec.name}-shape Q4_K_M greedy decode, bs=1, {args.ctx}-token context from a GPU "
                               f"prefill of seeded ids, {K} tokens"
                               + (", f16 KV cache" if args.kv == "f16" else ""), "ctx": args.ctx,
                   "decode_tokens": K, "batch": 1, "kv_cache": args.kv},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "roofline_tok": {"bytes_per_token": int(b_tok), "weight_bytes": int(w_bytes), "kv_bytes_f16": int(kv_bytes),
                         "roofline_tok_s": round(HBM_PEAK / b_tok, 1), "frac": round(frac_tok, 4)},
        "device_tok_s": round(K / dev_s, 2),
        "prefill_tok_s": round(args.ctx / prefill_s, 1) if prefill_s else None,
        "prefill": prefill,
        "other_kv_cache": other_kv,
        "kernels": prof or None,
        "gemv_microbench": micro,
        "tiny": tiny,
        "model_70b": model_70b,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark: batch-1 greedy decode of the synthetic Bonsai-27B-shape Q1_0 model on one MI355X.

Workload: 64-layer hybrid stack (48 Gated DeltaNet + 16 gated GQA
attention layers), random Q1_0 weights from include/daiza_synth.h, f16 embedding; a 1024-token
prefill of uniform-random ids, then `--steps` timed greedy decode tokens after `--warmup`
untimed ones.  One step = one token through the whole stack (forward_single_token).

Prints one JSON line.  `roofline` is the dominant kernel of the timed decode, the persistent token
kernel (one cooperative launch runs all timed tokens), timed with HIP events on the context's
stream: algorithmic bytes per launch (every token's Q1_0 weights, KV-cache reads and appends,
DeltaNet state read and write, conv ring, embedding row, logits) over the launch's duration; its
`traffic` is the HBM bytes per token of a profiled launch (profiles/decode_config4_pmc.txt) times
the timed launch's tokens.  `roofline_gemv` is a complete y = W x at the config-1 shape (17408 x
5120, 32 distinct matrices, more than the 256 MB Infinity Cache), timed per call.  `layer_steps`
times one mixer layer-step of configs 2 and 3 (at context 4096 and 32768).  `config5` times
speculative verify (k = 8 drafts at context 8192) after a batched prefill to
that context.  `cpu_baseline` is the CPU oracle (oracle/, a C restatement of the reference's
multithreaded AVX2 path) decoding a bounded sample from the GPU context's post-prefill state.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "batch-1 decode tok/s (27B-shape Q1_0 synth); Q1_0 GEMV HBM GB/s vs peak"
PEAK_GBS = 8000.0
SEED = 0xDA1A0004
PREFILL = 1024
VERIFY_CTX = 8192
VERIFY_K = 8


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def hip():
    h = ctypes.CDLL("libamdhip64.so")
    h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    h.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    h.hipDeviceSynchronize.argtypes = []
    h.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
    h.hipFree.argtypes = [ctypes.c_void_p]
    h.hipEventDestroy.argtypes = [ctypes.c_void_p]
    h.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    return h


class Events:
    def __init__(self, H, n):
        self.H = H
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            assert H.hipEventCreate(ctypes.byref(e)) == 0
            self.ev.append(e)

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        assert self.H.hipEventElapsedTime(ctypes.byref(ms), self.ev[a], self.ev[b]) == 0
        return ms.value

    def destroy(self):
        """Every HIP object this script creates is destroyed before exit (profilers that tear down
        after the program are sensitive to objects left alive)."""
        for e in self.ev:
            self.H.hipEventDestroy(e)
        self.ev = []


class Gate:
    """Holds a stream behind device-to-device copies (~1 ms each) while Python enqueues the timed
    work, so that no host-side enqueue gap falls inside a timed interval."""

    def __init__(self, H, s, n=16, nbytes=2 << 30):
        self.H = H
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        assert H.hipMalloc(ctypes.byref(self.a), nbytes) == 0 and H.hipMalloc(ctypes.byref(self.b), nbytes) == 0
        for _ in range(n):
            H.hipMemcpyAsync(self.b, self.a, nbytes, 3, s)

    def free(self):
        self.H.hipFree(self.a)
        self.H.hipFree(self.b)


def bench_copy(H, nbytes, reps=32):
    """Device-to-device copy of a known size: the reference point for the PMC byte counters and
    a copy-bandwidth ceiling measured in the same run."""
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    assert H.hipMalloc(ctypes.byref(a), nbytes) == 0 and H.hipMalloc(ctypes.byref(b), nbytes) == 0
    s = ctypes.c_void_p()
    H.hipStreamCreate(ctypes.byref(s))
    H.hipMemcpyAsync(b, a, nbytes, 3, s)
    H.hipStreamSynchronize(s)
    ev = Events(H, 2)
    g = Gate(H, s, n=4)
    H.hipEventRecord(ev.ev[0], s)
    for _ in range(reps):
        H.hipMemcpyAsync(b, a, nbytes, 3, s)
    H.hipEventRecord(ev.ev[1], s)
    H.hipEventSynchronize(ev.ev[1])
    g.free()
    us = 1e3 * ev.elapsed_ms(0, 1) / reps
    ev.destroy()
    H.hipStreamDestroy(s)
    H.hipFree(a)
    H.hipFree(b)
    return {"bytes": nbytes, "us": us, "gbs": 2 * nbytes / (us * 1e-6) / 1e9}


# Sources of each measured kernel: a PMC summary is used only for the source revision it was
# taken on (its `kernel_source_sha16:` line must equal the hash of these files in this tree).
KERNEL_SOURCES = {
    "decode_config4_pmc.txt": ["ptk_kernel.h", "ptk.h", "q1_gemv.h", "model_kernels.h", "common.h", "model.hip"],
    "gemv_config1_pmc.txt": ["q1_gemv.h", "common.h", "q1_mat.hip"],
}


def kernel_source_sha16(name):
    """sha256 prefix over the sources of the kernel a summary measures (file names and bytes)."""
    import hashlib
    h = hashlib.sha256()
    for f in KERNEL_SOURCES[name]:
        h.update(f.encode())
        with open(os.path.join(ROOT, "daiza_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic(name, key="traffic_bytes_per_launch"):
    """HBM bytes from a committed rocprofv3 --pmc summary under profiles/ (FETCH_SIZE and
    WRITE_SIZE, each scaled by the same counter on a copy of known size): the value of the line
    `key:`, or None when the summary or the line is absent, or when the summary was taken on other
    kernel sources than this tree's."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        if ":" in line and not line.startswith(" "):
            k, v = line.split(":", 1)
            vals[k.strip()] = v.strip()
    if vals.get("kernel_source_sha16") != kernel_source_sha16(name) or key not in vals:
        return None
    return int(float(vals[key]))


def decode_bytes(cfg, wbytes, pos0, n):
    """Algorithmic HBM bytes of n decode tokens at positions pos0 .. pos0+n-1: per token the Q1_0
    weights, the attention layers' KV reads over the context and K/V appends, the DeltaNet
    states read and written, the conv ring (3 history rows read, 1 written) and conv weights, the
    embedding row and the logits."""
    n_attn = sum(1 for i in range(cfg.n_layers) if (i + 1) % cfg.full_attn_interval == 0)
    n_ssm = cfg.n_layers - n_attn
    kv_row = 2 * cfg.n_head_kv * cfg.head_dim * 4           # K and V of one position, one layer
    state = cfg.ssm_v_heads * cfg.ssm_state * cfg.ssm_state * 4
    qkvd = cfg.qkv_dim
    per_tok = (wbytes + n_ssm * (2 * state + 4 * qkvd * 4 + 4 * qkvd * 4) + n_attn * kv_row
               + cfg.hidden * 2 + cfg.vocab * 4)
    ctx_rows = sum(pos0 + i + 1 for i in range(n))            # positions read, summed over tokens
    return n * per_tok + n_attn * kv_row * ctx_rows


def bench_verify(dz, H, ctx, cfg, decode_ms_per_tok, reps=8):
    """k = 8 uniform-random drafts verified in one forward at context 8192.
    Times dz_verify_forward (+ a commit of 0, so every rep sees the same context) with HIP events
    on the context's stream, and the full dz_spec_verify step at temperature 0.7 (Leviathan and
    bonus sampling on the host, logits copied back) by wall clock."""
    rng = np.random.default_rng(SEED & 0xFFF)
    t0 = time.time()
    while ctx.pos < VERIFY_CTX:
        n = min(1024, VERIFY_CTX - ctx.pos)
        ctx.forward_batch(rng.integers(0, cfg.vocab, n).astype(np.uint32))
    fill_s = time.time() - t0
    stream = ctypes.c_void_p(ctx.stream())
    ev = Events(H, 2)
    drafts = [rng.integers(0, cfg.vocab, VERIFY_K).astype(np.uint32) for _ in range(reps + 1)]
    ctx.verify_forward(drafts[0], want_logits=False)
    ctx.verify_commit(0)
    H.hipDeviceSynchronize()
    H.hipEventRecord(ev.ev[0], stream)
    for d in drafts[1:]:
        ctx.verify_forward(d, want_logits=False)
        ctx.verify_commit(0)
    H.hipEventRecord(ev.ev[1], stream)
    H.hipEventSynchronize(ev.ev[1])
    fwd_ms = ev.elapsed_ms(0, 1) / reps
    ev.destroy()
    params = dz.SamplingParams(0.7, 20, 0.95)
    lcg = dz.LcgRng(0xC0FFEE)
    dl = rng.standard_normal((VERIFY_K, cfg.vocab)).astype(np.float32)
    p0 = ctx.pos
    t0 = time.perf_counter()
    acc = 0
    for d in drafts[1:]:
        na, _ = ctx.spec_verify(d, dl, params, lcg)
        acc += na
    step_ms = 1e3 * (time.perf_counter() - t0) / reps
    return {
        "context": p0, "k": VERIFY_K, "temperature": 0.7,
        "verify_forward_ms": round(fwd_ms, 3),
        "spec_verify_step_ms": round(step_ms, 3),
        "sequential_verify_ms": round(VERIFY_K * decode_ms_per_tok, 3),
        "accepted_total": acc,
        "prefill_to_ctx_s": round(fill_s, 2),
        "note": "sequential_verify_ms = k forwards of one token on this build's decode path, the reference's "
                "verify loop (engine.rs:1255-1470); spec_verify_step_ms adds the device-side row statistics and top-k and the host draws (the draft logits' upload overlaps the forward on a side stream)",
    }


def bench_gemv(dz, H, rows=17408, cols=5120, nmat=32, reps=8):
    """HIP-event timing of a complete y = W x at the config-1 shape (dz_q1_0_matvec_dev: the split-K
    LUT GEMV and the tile sum that forms y) over a timed region of nmat*reps back-to-back calls on one
    stream, rotating nmat distinct matrices (more bytes than the 256 MB Infinity Cache).  Per-call
    time = region / calls; it includes the dispatch gaps, so it reads a little above the profiler's
    kernel durations."""
    # config-1 distribution: Bernoulli(0.5) sign bits, scale = f16(|N(0,1)| * 0.02), x ~ N(0,1)
    rng = np.random.default_rng(SEED)
    blk = np.empty((rows, cols // 128, 18), np.uint8)
    blk[:, :, 2:] = rng.integers(0, 256, (rows, cols // 128, 16), dtype=np.uint8)
    blk[:, :, :2] = (np.abs(rng.standard_normal((rows, cols // 128))) * 0.02).astype(np.float16)[..., None].view(np.uint8)
    aos = blk.reshape(-1)
    mats = [dz.Q1_0Matrix(aos, rows, cols) for _ in range(nmat)]
    x = rng.standard_normal(cols).astype(np.float32)
    L = dz.lib()
    dx, dy = ctypes.c_void_p(), ctypes.c_void_p()
    H.hipMalloc(ctypes.byref(dx), cols * 4)
    H.hipMalloc(ctypes.byref(dy), rows * 4)
    H.hipMemcpy(dx, x.ctypes.data, cols * 4, 1)
    s = ctypes.c_void_p()
    H.hipStreamCreate(ctypes.byref(s))
    for m in mats:  # warm-up (also sizes the library's partial buffer)
        assert L.dz_q1_0_matvec_dev(m._h, dx, dy, 0, s) == 0
    H.hipStreamSynchronize(s)
    # the result of the timed path against the oracle (one matrix, same x)
    import oracle
    y = np.empty(rows, np.float32)
    H.hipMemcpy(y.ctypes.data, dy, rows * 4, 2)
    yo = oracle.matvec(aos, rows, cols, x)
    rel = float(np.max(np.abs(y - yo)) / np.max(np.abs(yo)))
    n = nmat * reps
    ev = Events(H, 2)
    g = Gate(H, s)
    H.hipEventRecord(ev.ev[0], s)
    for i in range(n):
        L.dz_q1_0_matvec_dev(mats[i % nmat]._h, dx, dy, 0, s)
    H.hipEventRecord(ev.ev[1], s)
    H.hipEventSynchronize(ev.ev[1])
    g.free()
    if L.dz_q1_0_matvec_dev_status(s) != 0:  # a timed call whose wait gave up
        raise SystemExit("gemv: " + L.dz_last_error().decode())
    avg_us = 1e3 * ev.elapsed_ms(0, 1) / n
    algo = rows * (cols // 128) * 18 + cols * 4 + rows * 4  # W + x + y (config 1)
    ev.destroy()
    H.hipStreamDestroy(s)
    for m in mats:
        m.close()
    H.hipFree(dx)
    H.hipFree(dy)
    return {"avg_launch_us": avg_us, "launches": n, "algo_bytes": algo,
            "achieved_gbs": algo / (avg_us * 1e-6) / 1e9, "max_rel_err_vs_oracle": rel}


def layer_step_bytes(cfg, kind, ctx_len=0):
    """Algorithmic HBM bytes of one mixer layer-step (BASELINE configs 2 and 3): the Q1_0 weights of
    the in- and out-projections, plus for a DeltaNet layer the recurrent state read and written and
    the conv ring (3 history rows read, 1 written) with its weights, for an attention layer the K/V
    rows read over the context (the new position included) and the K/V append."""
    blk = lambda r, c: r * (c // 128) * 18
    H, hd = cfg.hidden, cfg.ssm_state
    if kind == "deltanet":
        inner, qkvd = cfg.ssm_v_heads * hd, cfg.qkv_dim
        w = blk(qkvd + inner + 2 * cfg.ssm_v_heads, H) + blk(H, inner)
        return w + 2 * cfg.ssm_v_heads * hd * hd * 4 + 4 * qkvd * 4 + 4 * qkvd * 4
    qd, kvd = cfg.n_head * cfg.head_dim, cfg.n_head_kv * cfg.head_dim
    w = blk(2 * qd + 2 * kvd, H) + blk(H, qd)
    return w + 2 * kvd * 4 * (ctx_len + 1) + 2 * kvd * 4


def bench_layers(dz, H, steps=40):
    """BASELINE configs 2 and 3 as isolated layer-steps: dz_ctx_mixer_step_dev (one mixer of one
    layer, h += mixer(rmsnorm(h)), weights, state and h resident in HBM) timed with HIP events on the
    context's stream over `steps` back-to-back steps.  Config 2: a 27B-shape Gated DeltaNet layer
    with N(0, 0.02) state and N(0, 0.1) conv history; config 3: a 27B-shape attention layer over an
    N(0,1) cache at context 4096 and 32768."""
    out = {}
    for name, L in (("config2_deltanet", 0), ("config3_attention_ctx4096", 4096),
                    ("config3_attention_ctx32768", 32768)):
        attn = L > 0
        cfg = dz.Config.bonsai27b(max_ctx=L + steps + 8)
        cfg.n_layers, cfg.vocab, cfg.full_attn_interval = 1, 1024, 1 if attn else 4
        model = dz.Model.synthetic(cfg, SEED + 2)
        ctx = dz.Context(model)
        rng = np.random.default_rng(L + 1)
        if attn:
            k = rng.standard_normal((cfg.n_head_kv, L, cfg.head_dim), dtype=np.float32)
            ctx.set_kv(0, k, k)
            del k
            ctx.set_pos(L)
        else:
            st = (rng.standard_normal((cfg.ssm_v_heads, cfg.ssm_state, cfg.ssm_state)) * 0.02).astype(np.float32)
            conv = (rng.standard_normal((4, cfg.qkv_dim)) * 0.1).astype(np.float32)
            ctx.set_ssm_state(0, st, conv, 0)
        h = rng.standard_normal(cfg.hidden).astype(np.float32)
        dh = ctypes.c_void_p()
        H.hipMalloc(ctypes.byref(dh), cfg.hidden * 4)
        H.hipMemcpy(dh, h.ctypes.data, cfg.hidden * 4, 1)
        Lb = dz.lib()
        stream = ctypes.c_void_p(ctx.stream())
        for _ in range(3):  # warm-up
            assert Lb.dz_ctx_mixer_step_dev(ctx._h, 0, dh, dh) == 0
        H.hipStreamSynchronize(stream)
        p0 = ctx.pos
        ev = Events(H, 2)
        g = Gate(H, stream, n=4)
        H.hipEventRecord(ev.ev[0], stream)
        for _ in range(steps):
            Lb.dz_ctx_mixer_step_dev(ctx._h, 0, dh, dh)
        H.hipEventRecord(ev.ev[1], stream)
        H.hipEventSynchronize(ev.ev[1])
        g.free()
        us = 1e3 * ev.elapsed_ms(0, 1) / steps
        ev.destroy()
        kind = "attention" if attn else "deltanet"
        algo = sum(layer_step_bytes(cfg, kind, p0 + i) for i in range(steps)) / steps
        out[name] = {"us_per_step": round(us, 2), "algo_bytes_per_step": int(algo),
                     "achieved_gbs": round(algo / (us * 1e-6) / 1e9, 1),
                     "frac": round(algo / (us * 1e-6) / 1e9 / PEAK_GBS, 4),
                     "context": p0 if attn else None}
        log("%s: %.2f us per layer-step, %.1f GB/s" % (name, us, out[name]["achieved_gbs"]))
        H.hipFree(dh)
        ctx.close()
        model.close()
    return out


def snapshot_state(ctx, cfg):
    """Host copies of every layer's state of a context (DeltaNet state, conv ring and head; K/V of
    the cached positions), for the CPU baseline to start from the GPU's prefill."""
    snap = {"pos": ctx.pos, "ssm": {}, "kv": {}}
    for l in range(cfg.n_layers):
        if (l + 1) % cfg.full_attn_interval:
            snap["ssm"][l] = ctx.get_ssm_state(l)
        else:
            snap["kv"][l] = ctx.get_kv(l, ctx.pos)
    return snap


def cpu_baseline(cfg_cls, snap, first, budget_s=20.0):
    """Oracle (C restatement of the reference AVX2 path: quad LUT kernel, work-stealing 128-row
    chunks) greedy decode on the host cores, from the GPU context's state after the same
    1024-token prefill (copied in: the oracle's own token-by-token prefill would take minutes)."""
    import oracle
    # the GPU box grants 16 host CPUs per GPU
    threads = min(os.cpu_count() or 1, int(os.environ.get("DZ_CPU_THREADS", 16)))
    cfg = cfg_cls.bonsai27b(max_ctx=snap["pos"] + 80)
    t0 = time.time()
    om = oracle.Model(cfg, SEED, nthreads=threads)
    gen_s = time.time() - t0
    om.set_pos(snap["pos"])
    for l, (st, conv, head) in snap["ssm"].items():
        om.set_ssm_state(l, st, conv, head)
    for l, (k, v) in snap["kv"].items():
        om.set_kv(l, k, v)
    tok = first
    n = 0
    t0 = time.time()
    while True:
        tok, _ = om.forward(tok, want_logits=False)
        n += 1
        el = time.time() - t0
        if el > budget_s or n >= 64:
            break
    om.close()
    model = "unknown CPU"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": n / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": "oracle greedy decode of %d tokens at context %d-%d (the GPU context's state after the same "
                      "%d-token prefill, copied in), full 27B shape, %d threads on %s (%d logical CPUs visible; "
                      "model generation %.1f s excluded)"
                      % (n, snap["pos"], snap["pos"] + n, snap["pos"], threads, model, os.cpu_count() or 0, gen_s)}


def trace_decode(dz, args):
    """--only trace: the prefill and one decode launch through library calls alone, timed by the host
    clock, for rocprofv3 passes.  Everything is closed before return; with --maps the process's
    memory map is written first (to symbolize an exit-time stack)."""
    cfg = dz.Config.bonsai27b(max_ctx=args.prefill + args.warmup + args.steps + 8)
    model = dz.Model.synthetic(cfg, SEED)
    ctx = dz.Context(model)
    prompt = np.random.default_rng(SEED & 0xFFFF).integers(0, cfg.vocab, args.prefill).astype(np.uint32)
    t0 = time.perf_counter()
    last = ctx.forward_batch(prompt)
    print("[trace] prefill %d tokens in %.3f s" % (args.prefill, time.perf_counter() - t0), flush=True)
    toks = ctx.decode_greedy(int(np.argmax(last)), max(1, args.warmup))
    t0 = time.perf_counter()
    ctx.decode_greedy(int(toks[-1]), args.steps)
    dt = time.perf_counter() - t0
    print("[trace] decode %d tokens in one launch: %.2f tok/s (host clock)" % (args.steps, args.steps / dt), flush=True)
    if args.maps:
        with open("/proc/self/maps") as f, open(args.maps, "w") as o:
            o.write(f.read())
    ctx.close()
    model.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prefill", type=int, default=PREFILL)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--maps", default="", help="--only trace: write /proc/self/maps to this file")
    ap.add_argument("--only", choices=["all", "gemv", "decode", "verify", "layers", "trace"], default="all",
                    help="gemv: only the config-1 GEMV and the copy reference; decode: only the prefill, the "
                         "timed decode and a 256 MiB copy reference; verify: only the config-5 verify; layers: "
                         "only the config-2/3 layer-steps; trace: the "
                         "prefill and decode through library calls alone, timed by the host clock (for "
                         "rocprofv3 passes, which lose their output when the script's own HIP objects exist)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build runs the decode loop on a single GPU "
              "(this build has no multi-GPU path); use --gpus 1", file=sys.stderr)
        return 2

    import daiza_amd as dz
    if args.only == "trace":
        trace_decode(dz, args)
        return 0
    H = hip()
    L = dz.lib()
    if L.dz_device_init(0) != 0:
        raise SystemExit("dz_device_init: " + L.dz_last_error().decode())
    if args.only == "layers":
        bench_layers(dz, H)
        return 0
    if args.only == "gemv":
        g = bench_gemv(dz, H)
        cp = bench_copy(H, g["algo_bytes"])
        log("gemv: %.2f us per launch, %.1f GB/s; copy of %d B: %.2f us, %.1f GB/s"
            % (g["avg_launch_us"], g["achieved_gbs"], cp["bytes"], cp["us"], cp["gbs"]))
        return 0

    max_ctx = max(args.prefill + 2 * (args.warmup + args.steps) + 8, VERIFY_CTX + 4 * VERIFY_K * 4)
    cfg = dz.Config.bonsai27b(max_ctx=max_ctx)
    if args.only == "verify":
        model = dz.Model.synthetic(cfg, SEED)
        ctx = dz.Context(model)
        v = bench_verify(dz, H, ctx, cfg, float("nan"))
        log("config 5: verify forward %.2f ms, spec step %.2f ms at context %d"
            % (v["verify_forward_ms"], v["spec_verify_step_ms"], v["context"]))
        ctx.close()
        model.close()
        H.hipDeviceSynchronize()
        return 0
    t0 = time.time()
    log("building synthetic 27B-shape model")
    model = dz.Model.synthetic(cfg, SEED)
    build_s = time.time() - t0
    log("model built in %.1f s" % build_s)
    ctx = dz.Context(model)
    wbytes = model.q1_bytes()

    rng = np.random.default_rng(SEED & 0xFFFF)
    prompt = rng.integers(0, cfg.vocab, args.prefill).astype(np.uint32)
    t0 = time.time()
    last = ctx.forward_batch(prompt)
    prefill_s = time.time() - t0
    log("prefill %d tokens in %.2f s" % (args.prefill, prefill_s))
    first = int(np.argmax(last))
    snap = None if args.no_cpu or args.only != "all" else snapshot_state(ctx, cfg)

    stream = ctypes.c_void_p(ctx.stream())
    ev = Events(H, 2)
    toks_w = ctx.decode_greedy(first, args.warmup) if args.warmup else np.array([first], np.uint32)
    nxt = int(toks_w[-1])
    H.hipDeviceSynchronize()
    H.hipEventRecord(ev.ev[0], stream)
    t0 = time.perf_counter()
    toks = ctx.decode_greedy(nxt, args.steps)
    H.hipEventRecord(ev.ev[1], stream)
    H.hipEventSynchronize(ev.ev[1])
    H.hipDeviceSynchronize()
    wall = time.perf_counter() - t0
    ms = ev.elapsed_ms(0, 1)
    ev.destroy()
    tps = args.steps / (ms / 1e3)
    decode_ctx_end = ctx.pos  # before the sampled run and the config-5 verify continue on this context

    log("decode %d tokens: %.2f tok/s" % (args.steps, tps))
    pos_timed = args.prefill + args.warmup
    algo = decode_bytes(cfg, wbytes, pos_timed, args.steps)
    ptk_gbs = algo / (ms * 1e-3) / 1e9
    # HBM bytes of the timed launch: the profiled launch's bytes per token times this launch's tokens
    per_tok = measured_traffic("decode_config4_pmc.txt", "traffic_bytes_per_token")
    ptk_traffic = per_tok * args.steps if per_tok else None
    if args.only == "decode":
        cp = bench_copy(H, 256 << 20, reps=4)
        log("token kernel: %.1f GB/s algorithmic over %.1f ms (%d B per launch); copy of %d B: %.1f GB/s"
            % (ptk_gbs, ms, algo, cp["bytes"], cp["gbs"]))
        ctx.close()
        model.close()
        H.hipDeviceSynchronize()
        return 0
    # the same loop with the reference's default sampling (T 0.7, top-k 20, top-p 0.95) drawn on the
    # device inside the token kernel (dz_decode_sample): the rate a non-greedy caller gets
    smp = dz.SamplingParams(0.7, 20, 0.95)
    srng = dz.LcgRng(SEED & 0xFFFFFFFF)
    ev = Events(H, 2)
    stoks = ctx.decode_sample(int(toks[-1]), max(1, args.warmup), smp, srng)
    H.hipDeviceSynchronize()
    H.hipEventRecord(ev.ev[0], stream)
    ctx.decode_sample(int(stoks[-1]), args.steps, smp, srng)
    H.hipEventRecord(ev.ev[1], stream)
    H.hipEventSynchronize(ev.ev[1])
    sms = ev.elapsed_ms(0, 1)
    ev.destroy()
    sampled = {"tok_s": round(args.steps / (sms / 1e3), 2), "ms_per_token": round(sms / args.steps, 4),
               "tokens": args.steps, "temperature": 0.7, "top_k": 20, "top_p": 0.95,
               "context_at_end": ctx.pos}
    log("sampled decode %d tokens: %.2f tok/s" % (args.steps, sampled["tok_s"]))
    g = bench_gemv(dz, H)
    cp = bench_copy(H, g["algo_bytes"])
    log("gemv: %.2f us per launch; copy ceiling %.1f GB/s" % (g["avg_launch_us"], cp["gbs"]))
    v = bench_verify(dz, H, ctx, cfg, ms / args.steps)
    log("config 5: verify forward %.2f ms, spec step %.2f ms (sequential %.2f ms) at context %d"
        % (v["verify_forward_ms"], v["spec_verify_step_ms"], v["sequential_verify_ms"], v["context"]))
    ctx.close()
    model.close()
    layers = bench_layers(dz, H)
    out = {
        "metric": METRIC,
        "value": round(tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE config 4: Bonsai-27B-shape synthetic Q1_0 (64 layers: 48 Gated DeltaNet + 16 gated "
                        "GQA attention, hidden 5120, FFN 17408, vocab 248320, f16 embedding), %d-token random prefill, "
                        "then greedy decode" % args.prefill,
            "prefill_tokens": args.prefill,
            "decode_tokens": args.steps,
            "context_at_end": decode_ctx_end,
            "q1_weight_bytes_per_token": wbytes,
            "weight_roofline_tok_s": round(PEAK_GBS * 1e9 / wbytes, 1),
            "weight_roofline_frac": round(tps * wbytes / (PEAK_GBS * 1e9), 4),
            "prefill_s": round(prefill_s, 3),
            "model_build_s": round(build_s, 1),
            "decode_wall_s": round(wall, 4),
        },
        "roofline": {
            "kernel": "ptk_kernel (persistent token kernel: %d decode tokens per launch)" % args.steps,
            "bound": "hbm",
            "achieved": round(ptk_gbs, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(ptk_gbs / PEAK_GBS, 4),
            "traffic": ptk_traffic,
            "avg_launch_us": round(ms * 1e3, 1),
            "launches_timed": 1,
            "algo_bytes_per_launch": algo,
            "copy_ceiling_gbs": round(cp["gbs"], 1),
        },
        "roofline_gemv": {
            "kernel": "dz_q1_0_matvec_dev (Q1_0 LUT GEMV, config 1 17408x5120: complete y = W x)",
            "bound": "hbm",
            "achieved": round(g["achieved_gbs"], 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(g["achieved_gbs"] / PEAK_GBS, 4),
            "traffic": measured_traffic("gemv_config1_pmc.txt", "traffic_bytes_per_call"),
            "avg_launch_us": round(g["avg_launch_us"], 3),
            "max_rel_err_vs_oracle": g["max_rel_err_vs_oracle"],
            "launches_timed": g["launches"],
            "algo_bytes_per_launch": g["algo_bytes"],
        },
        "sampled_decode": sampled,
        "config5": v,
        "layer_steps": layers,
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(dz.Config, snap, first, args.cpu_budget)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    # a zero status ends the script normally (no SystemExit): rocprofv3 then writes its output
    # before the runtime's teardown
    _rc = main()
    if _rc:
        sys.exit(_rc)

"""Benchmark: GPT 12L/d768 training step on one MI355X.

One step = the reference train step (src/text_train.cpp:1181-1330) on the HIP
engine: GPTModel forward (ALiBi, materialised attention), sparse cross-entropy
with the loss downloaded, backward, one AdamW update, zero_grad. Inputs
(weights N(0,0.02), biases 0, gains 1, tokens U[0,32000)) are synthetic, seeded,
and resident in device memory before timing starts.

Prints one JSON line. `roofline` covers the dominant kernel family (the fp32
MFMA GEMMs: every matmul / batched_matmul launch of the timed steps, timed with
HIP events on the engine's stream). `attention` reports the metric's second
part: the fused causal-attention primitives on BASELINE config 2 (forward:
bmm_reduce Max -> softmax_denom -> softmax_apply) and config 5 (document-masked
forward + backward over the 8 packed rows), as algorithmic TFLOP/s (4*d*P
forward, 8*d*P backward over the P allowed (query, key) pairs) and as a
fraction of the fp32 MFMA peak, timed with HIP events on the engine's stream
at a steady clock (0.25 s of untimed calls first, then at least 20 ms timed).
`cpu_baseline` runs the CPU restatement of the reference CpuEngine (oracle/,
loaded only for this leg) on a bounded sample of the same workload: the
config-4 model at batch 1 of 8, one warmup and three timed training steps.
`--cpu-legs` runs the oracle's legs of configs 2, 3 and 5 instead.
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "neuralnet.cpp_amd"))

CFG = dict(vocab_size=32000, d_model=768, seq_len=1024, num_heads=12, d_ff=3072, num_layers=12, pos_enc="alibi")
BATCH = 8
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def step_flops(cfg, batch):
    """Algorithmic FLOPs of one step: 6*P_mm*N + 12*L*H*d*P_attn*B, P_attn = T(T+1)/2."""
    D, F, V, L, T, H = (cfg[k] for k in ("d_model", "d_ff", "vocab_size", "num_layers", "seq_len", "num_heads"))
    p_mm = L * (4 * D * D + D * 2 * F + F * D) + D * V
    n = batch * T
    p_attn = T * (T + 1) // 2
    return 6 * p_mm * n + 12 * L * H * (D // H) * p_attn * batch


def init_session(eng, cfg, batch, seed):
    g = eng.gpt(**cfg)
    rng = np.random.default_rng(seed)
    shapes = g.param_shapes()
    params = [None] * len(shapes)
    gains = set(_gain_indices(cfg))
    for i, (r, c) in enumerate(shapes):
        if i in gains:
            params[i] = np.ones((r, c), dtype=np.float32)
        elif c == 1:
            params[i] = np.zeros((r, c), dtype=np.float32)           # biases
        else:
            params[i] = (rng.standard_normal((r, c), dtype=np.float32) * np.float32(0.02))
    g.set_params(params)
    T = cfg["seq_len"]
    toks = rng.integers(0, cfg["vocab_size"], size=(T + 1, batch))
    g.load_batch(toks[:T].astype(np.float32), toks[1:].T.reshape(-1))
    return g


def _gain_indices(cfg):
    base = 2 if cfg["pos_enc"] == "learned" else 1
    idx = []
    for layer in range(cfg["num_layers"]):
        idx += [base + 14 * layer + 8, base + 14 * layer + 13]
    return idx + [base + 14 * cfg["num_layers"]]


# The config-4 step's main product shapes as C (M, N) = op(A) op(B) over K, with the engine's transposes.
LIBRARY_SHAPES = [(6144, 8192, 768, False, False), (768, 8192, 3072, False, False), (768, 8192, 6144, True, False),
                  (3072, 8192, 768, True, False), (6144, 768, 8192, False, True), (768, 3072, 8192, False, True),
                  (768, 768, 8192, False, True), (768, 8192, 768, False, False), (32000, 8192, 768, False, False),
                  (768, 8192, 32000, True, False), (4096, 4096, 4096, False, False)]


def library_gemm_leg(reps=30):
    """torch.mm in fp32 (TF32 off: ROCm's vendor GEMM) on the step's shapes, 10 untimed then `reps` timed
    calls between torch.cuda events: a reference point for the engine's own kernels (roofline.by_shape)."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    out = []
    for M, N, K, ta, tb in LIBRARY_SHAPES:
        A = torch.randn((K, M) if ta else (M, K), device=dev, generator=gen)
        B = torch.randn((N, K) if tb else (K, N), device=dev, generator=gen)
        a, b = (A.t() if ta else A), (B.t() if tb else B)
        C = torch.empty((M, N), device=dev)
        for _ in range(10):
            torch.mm(a, b, out=C)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            torch.mm(a, b, out=C)
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e) / reps
        out.append(dict(M=M, N=N, K=K, transA=int(ta), transB=int(tb), ms=ms, tflops=2 * M * N * K / ms / 1e9,
                        frac_of_fp32_mfma_peak=2 * M * N * K / ms / 1e9 / PEAK_FP32_MFMA_TFLOPS))
        del A, B, C
    return out


def inference_leg(g, seed, tokens=64, warmup=8):
    """Incremental inference on the trained config-4 model (GPTModel::forward_step with KV caches,
    reference compute_layer.hpp:2906-2960): one token per call at positions 0..tokens-1, logits
    (32000 floats) copied to the host after each, so a call is one token's full latency."""
    rng = np.random.default_rng(seed + 17)
    ids = rng.integers(0, CFG["vocab_size"], size=warmup + tokens)
    g.reset_cache()
    for p in range(warmup):
        g.forward_step(int(ids[p]), p, p)
    t0 = time.perf_counter()
    for p in range(warmup, warmup + tokens):
        g.forward_step(int(ids[p]), p, p)
    el = time.perf_counter() - t0
    g.reset_cache()
    return {"tokens": tokens, "positions": [warmup, warmup + tokens - 1], "ms_per_token": 1000.0 * el / tokens,
            "tokens_per_s": tokens / el,
            "workload": "config-4 model, batch 1, one token per forward_step (KV caches), logits read back"}


def gpu_leg(steps, warmup, seed, inference=True):
    import nnengine
    lib = nnengine.hip_library()
    eng = nnengine.Engine(lib)
    lib.nnhip_engine_profile_gemm.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.nnhip_engine_profile_gemm_read.argtypes = [ctypes.c_void_p] + [ctypes.POINTER(ctypes.c_double)] * 3
    t0 = time.perf_counter()
    g = init_session(eng, CFG, BATCH, seed)
    print(f"[bench] model ready in {time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)
    losses = []
    for i in range(warmup):
        losses.append(g.train_step())
        print(f"[bench] warmup step {i} loss {losses[-1]:.4f}", file=sys.stderr, flush=True)
    eng.sync()
    eng._check(lib.nnhip_engine_profile_gemm(eng._e, 1))
    t0 = time.perf_counter()
    for i in range(steps):
        losses.append(g.train_step())
    eng.sync()
    elapsed = time.perf_counter() - t0
    lib.nnhip_engine_profile_gemm_records.restype = ctypes.c_long
    lib.nnhip_engine_profile_gemm_records.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double),
                                                      ctypes.c_size_t]
    cap = 1 << 16
    buf = (ctypes.c_double * (7 * cap))()
    n = lib.nnhip_engine_profile_gemm_records(eng._e, buf, cap)
    if n < 0:
        raise RuntimeError("GEMM profile read failed")
    rec = np.frombuffer(buf, dtype=np.float64, count=7 * n).reshape(n, 7)
    eng._check(lib.nnhip_engine_profile_gemm(eng._e, 0))
    by_shape = {}
    for M, N, K, b, ta, tb, t in rec:
        key = (int(M), int(N), int(K), int(b), int(ta), int(tb))
        e = by_shape.setdefault(key, [0, 0.0])
        e[0] += 1
        e[1] += t
    shapes = []
    for (M, N, K, b, ta, tb), (cnt, t) in sorted(by_shape.items(), key=lambda kv: -kv[1][1]):
        fl = 2.0 * M * N * K * b
        shapes.append({"M": M, "N": N, "K": K, "batch": b, "transA": ta, "transB": tb,
                       "launches_per_step": cnt / steps, "ms_per_step": t / steps,
                       "tflops": fl / (t / cnt * 1e-3) / 1e12})
    launches = ctypes.c_double(float(n))
    flops = ctypes.c_double(float((2.0 * rec[:, 0] * rec[:, 1] * rec[:, 2] * rec[:, 3]).sum()))
    ms = ctypes.c_double(float(rec[:, 6].sum()))
    print(f"[bench] timed {steps} steps in {elapsed:.3f}s, losses {[round(x, 4) for x in losses]}",
          file=sys.stderr, flush=True)
    infer = inference_leg(g, seed) if inference else None
    for x in losses:
        if not math.isfinite(x):
            raise RuntimeError(f"non-finite loss {x}")
    return dict(elapsed=elapsed, inference=infer, gemm_launches=launches.value, gemm_flops=flops.value,
                gemm_ms=ms.value,
                losses=losses, gemm_shapes=shapes)


class StreamTimer:
    """HIP events recorded on the engine's stream (the HIP runtime libnnhip.so links)."""

    def __init__(self, lib, eng):
        self.hip = ctypes.CDLL("libamdhip64.so")
        lib.nnhip_engine_stream.restype = ctypes.c_void_p
        lib.nnhip_engine_stream.argtypes = [ctypes.c_void_p]
        self.stream = ctypes.c_void_p(lib.nnhip_engine_stream(eng._e))
        self.ev = [ctypes.c_void_p(), ctypes.c_void_p()]
        for e in self.ev:
            self._ok(self.hip.hipEventCreate(ctypes.byref(e)))

    def _ok(self, rc):
        if rc != 0:
            raise RuntimeError(f"HIP error {rc}")

    def start(self):
        self._ok(self.hip.hipEventRecord(self.ev[0], self.stream))

    def stop_ms(self):
        self._ok(self.hip.hipEventRecord(self.ev[1], self.stream))
        self._ok(self.hip.hipEventSynchronize(self.ev[1]))
        ms = ctypes.c_float()
        self._ok(self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[0], self.ev[1]))
        return ms.value


class Busy:
    """Keeps the GPU busy while the host queues short kernels: 4096^3 GEMMs
    covering `ms` milliseconds are enqueued before the start event, so the
    launches that follow run back to back and the event interval measures
    kernel time, not host submission rate."""

    def __init__(self, eng, rng):
        self.eng = eng
        self.a = eng.tensor(rng.uniform(-1, 1, (4096, 4096)).astype(np.float32))
        self.gemm_ms = None

    def _gemm(self):
        c = self.eng.matmul(self.a, self.a)
        self.eng.settle()   # matmul is recorded until its result is used: launch it now
        del c

    def __call__(self, ms=3.0):
        if self.gemm_ms is None:
            self._gemm()
            self.eng.sync()
            t0 = time.perf_counter()
            for _ in range(4):
                self._gemm()
            self.eng.sync()
            self.gemm_ms = (time.perf_counter() - t0) * 1e3 / 4
        for _ in range(max(2, math.ceil(ms / self.gemm_ms))):
            self._gemm()


def timed_ms(timer, busy, fn, reps, warmup=3, steady=True, warm_s=0.25, min_ms=20.0):
    """Average milliseconds per call of fn over back-to-back calls. steady
    (compute-bound calls): after untimed calls for at least `warmup` calls and
    warm_s seconds, over at least `reps` calls and min_ms of work, since the
    GPU raises its clock only after a while under load (a config-2 forward
    measured 63 TFLOP/s cold and 79 after a second of work) and short timed
    regions would report the ramp. Otherwise (the short memory-bound kernels):
    `warmup` untimed calls, then `reps` timed calls behind ~3 ms of GEMMs. The
    engine records some calls instead of launching them and skips results that
    nobody references, so each call's outputs are held until settle() has
    launched what the call recorded, then dropped (the pool hands the same
    block to the next call)."""
    def call():
        keep = fn()
        busy.eng.settle()
        del keep

    if not steady:
        for _ in range(warmup):
            call()
        busy()
        timer.start()
        for _ in range(reps):
            call()
        return timer.stop_ms() / reps

    t0, n = time.perf_counter(), 0
    while n < warmup or time.perf_counter() - t0 < warm_s:
        call()
        n += 1
        if n % 8 == 0:
            busy.eng.sync()   # keep the host within a few calls of the GPU
    busy.eng.sync()
    # Host cost of queueing one call (measured behind GEMMs that keep the GPU
    # busy) and an upper bound of its GPU time (host and GPU serialised).
    busy(6.0)
    t1 = time.perf_counter()
    for _ in range(4):
        call()
    host_ms = (time.perf_counter() - t1) * 1e3 / 4
    busy.eng.sync()
    t2 = time.perf_counter()
    for _ in range(4):
        call()
    busy.eng.sync()
    gpu_ms = (time.perf_counter() - t2) * 1e3 / 4
    reps = max(reps, min(2000, math.ceil(min_ms / max(gpu_ms, 1e-3))))
    busy(1.25 * reps * host_ms + 2.0)
    timer.start()
    for _ in range(reps):
        keep = fn()
        busy.eng.settle()
        del keep
    return timer.stop_ms() / reps


def attention_leg(seed, reps=5):
    """BASELINE configs 2 and 5 through the engine's fused attention primitives."""
    import nnengine
    lib = nnengine.hip_library()
    eng = nnengine.Engine(lib)
    timer = StreamTimer(lib, eng)
    rng = np.random.default_rng(seed)
    busy = Busy(eng, rng)
    out = {}

    # config 2: B 16 x H 8 = 128 heads, T 512, d 64, causal, alpha 1/8.
    BH, T, d = 128, 512, 64
    q, k = (eng.tensor(rng.standard_normal((BH * d, T), dtype=np.float32)) for _ in range(2))
    vt = eng.tensor(rng.standard_normal((BH * T, d), dtype=np.float32))
    mask = eng.tensor(eng.build_attention_mask(1, T, 1, False))

    def fwd():
        m = eng.batched_matmul_reduce(q, k, BH, "Max", True, False, 0.125, True, mask)
        l = eng.batched_matmul_softmax_denom(q, k, m, BH, True, False, 0.125, mask)
        return eng.batched_matmul_softmax_apply(q, k, vt, m, l, BH, True, False, 0.125, mask)
    ms = timed_ms(timer, busy, fwd, reps)
    flop = 4 * d * (T * (T + 1) // 2) * BH
    out["causal_config2_forward"] = {
        "tflops": flop / (ms * 1e-3) / 1e12, "frac_of_fp32_mfma_peak": flop / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
        "ms": ms, "flop": flop, "dense_equivalent_tflops": 4 * d * T * T * BH / (ms * 1e-3) / 1e12,
        "workload": "B16 x H8, T512, d64, causal mask, alpha 1/8: bmm_reduce(Max) + softmax_denom + softmax_apply"}
    del q, k, vt, mask

    # config 5: B 8, H 12, T 2048, d 64; documents U{64..1024} per row, blocked across boundaries.
    B, H, T = 8, 12, 2048
    rows = []
    pairs = 0
    for _ in range(B):
        lens, tot = [], 0
        while tot < T:
            L = min(int(rng.integers(64, 1025)), T - tot)
            lens.append(L)
            tot += L
        ids = np.concatenate([np.full(L, i + 1, dtype=np.uint64) for i, L in enumerate(lens)])
        pairs += sum(L * (L + 1) // 2 for L in lens)
        mk = eng.tensor(eng.build_attention_mask(1, T, 1, False, doc_ids=ids))
        rows.append([eng.tensor(rng.standard_normal((H * d, T), dtype=np.float32)) for _ in range(4)] + [mk])

    def row(q, k, v, g, mk):
        # The reference's call sequence for one packed row (compute_layer.hpp:1196-1221, :1304-1327);
        # its temporaries (the dP product among them) end with the call, as in the layer. The engine
        # records each row's fused forward and backward and launches the rows together.
        m = eng.batched_matmul_reduce(q, k, H, "Max", True, False, 0.125, True, mk)
        l = eng.batched_matmul_softmax_denom(q, k, m, H, True, False, 0.125, mk)
        vt = eng.rearrange_3d(eng.transpose(v), T, H, d)
        o = eng.batched_matmul_softmax_apply(q, k, vt, m, l, H, True, False, 0.125, mk)
        P = eng.batched_matmul(g, v, H, True, False)
        G = eng.rearrange_3d(eng.transpose(g), T, H, d)
        dq, r = eng.batched_matmul_softmax_backward_q(q, k, P, m, l, H, True, False, 0.125, mk)
        dk, dv = eng.batched_matmul_softmax_backward_kv(q, k, P, G, r, m, l, H, True, False, 0.125, mk)
        return o, dq, dk, dv

    def fwd_bwd():
        # every row's outputs stay referenced until the call is settled, as a caller keeps them
        return [row(q, k, v, g, mk) for q, k, v, g, mk in rows]
    ms = timed_ms(timer, busy, fwd_bwd, reps)
    flop = 12 * d * pairs * H
    out["doc_masked_config5_forward_backward"] = {
        "tflops": flop / (ms * 1e-3) / 1e12, "frac_of_fp32_mfma_peak": flop / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
        "ms": ms, "flop": flop, "allowed_pair_fraction": pairs / (B * T * T),
        "workload": "B8 x H12, T2048, d64, doc lengths U{64..1024}: forward (reduce, denom, apply) + dP GEMM + "
                    "backward_q + backward_kv, all 8 rows"}
    eng.sync()
    return out


# GEMM sweep (A (M,K) x B (K,N), NN) plus the GPT-shaped
# Linear products of config 4 in the reference's orientation (W (out,in) x X
# (in, tokens)) and their backward variants (dX = W^T G: TN, dW = G X^T: NT).
GEMM_SWEEP = [
    ("square 1024", 1024, 1024, 1024, False, False),
    ("square 2048", 2048, 2048, 2048, False, False),
    ("square 4096", 4096, 4096, 4096, False, False),
    ("QKV [8192x768]x[768x2304]", 8192, 768, 2304, False, False),
    ("FFN up [8192x768]x[768x3072]", 8192, 768, 3072, False, False),
    ("FFN down [8192x3072]x[3072x768]", 8192, 3072, 768, False, False),
    ("Linear fwd fc1 W(6144,768) X(768,8192)", 6144, 768, 8192, False, False),
    ("Linear fwd fc2 W(768,3072) X(3072,8192)", 768, 3072, 8192, False, False),
    ("Linear fwd lm_head W(32000,768) X(768,8192)", 32000, 768, 8192, False, False),
    ("Linear bwd dX fc1 W^T G (TN)", 768, 6144, 8192, True, False),
    ("Linear bwd dW fc1 G X^T (NT)", 6144, 8192, 768, False, True),
    ("Linear bwd dX lm_head W^T G (TN)", 768, 32000, 8192, True, False),
    ("Linear bwd dW lm_head G X^T (NT)", 32000, 8192, 768, False, True),
]


def gemm_leg(seed):
    import nnengine
    lib = nnengine.hip_library()
    eng = nnengine.Engine(lib)
    timer = StreamTimer(lib, eng)
    rng = np.random.default_rng(seed)
    busy = Busy(eng, rng)
    out = []
    for name, M, K, N, tA, tB in GEMM_SWEEP:
        a = eng.tensor(rng.uniform(-1, 1, (K, M) if tA else (M, K)).astype(np.float32))
        b = eng.tensor(rng.uniform(-1, 1, (N, K) if tB else (K, N)).astype(np.float32))
        flop = 2.0 * M * N * K
        reps = max(3, min(50, int(2e12 / flop)))
        ms = timed_ms(timer, busy, lambda: eng.matmul(a, b, tA, tB), reps)
        tf = flop / (ms * 1e-3) / 1e12
        out.append({"shape": name, "M": M, "N": N, "K": K, "transA": tA, "transB": tB, "ms": ms, "tflops": tf,
                    "frac_of_fp32_mfma_peak": tf / PEAK_FP32_MFMA_TFLOPS})
        del a, b
    eng.sync()
    return out


def hbm_leg(seed):
    """Memory-bound kernels on the config-4 tensors: algorithmic bytes (distinct
    inputs read + outputs written, fp32) per call / kernel time. Each case cycles
    through copies of its inputs that together exceed 768 MB, so consecutive
    calls do not find their inputs in the 256 MB Infinity Cache."""
    import nnengine
    import layer_programs as lp
    lib = nnengine.hip_library()
    eng = nnengine.Engine(lib)
    timer = StreamTimer(lib, eng)
    rng = np.random.default_rng(seed)
    busy = Busy(eng, rng)
    F, N, FF, R, C, V = 768, 8192, 3072, 98304, 1024, 32000

    def h(shape, lo=-1.0, hi=1.0):
        return rng.uniform(lo, hi, shape).astype(np.float32)

    host = dict(x=h((F, N)), g=h((F, N)), normed=h((F, N)), gamma=h((F, 1), 0.5, 1.5), rinv=h((1, N), 0.5, 2.0),
                mvec=h((1, N)), gate=h((FF, N)), up=h((FF, N)), s=h((FF, N), 0.0, 1.0), gff=h((FF, N)),
                scores=h((R, C), -4.0, 4.0), sg=h((R, C)), logits=h((V, N), -3.0, 3.0),
                labels=rng.integers(0, V, (1, N)).astype(np.float32), table=h((V, F)),
                idx=rng.integers(0, V, (N, 1)).astype(np.float32), grad_rows=h((N, F)),
                mask=np.tile(np.triu(np.full((C, C), -np.inf, np.float32), 1), (R // C, 1)))
    host["gate2"] = np.concatenate([host["gate"], host["up"]])   # fc1's (6144, 8192) output gradient

    def prog(name, vec=False):
        spec, _ = getattr(lp, name)()
        return lambda args, rows, cols: (eng.eval_expr_reduce if vec else eng.eval_expr)(spec, args, rows, cols)

    fn, fb, bb = F * N * 4, FF * N * 4, R * C * 4
    # (name, input names, call(tensors) -> result, algorithmic bytes)
    cases = [
        ("RMSNorm fwd sum of squares ColSum(x*x) (768x8192)", ["x"],
         lambda t: prog("rms_sum_sq", True)([t["x"], t["x"]], F, N), fn + N * 4),
        ("RMSNorm fwd x*colbcast(rinv) (768x8192)", ["x", "rinv"],
         lambda t: prog("rms_normalize")([t["x"], t["rinv"]], F, N), 2 * fn + N * 4),
        ("RMSNorm fwd normed*rowbcast(gamma) (768x8192)", ["normed", "gamma"],
         lambda t: prog("rms_scale")([t["normed"], t["gamma"]], F, N), 2 * fn + F * 4),
        ("RMSNorm bwd ColSum(g*gamma*normed) (768x8192)", ["g", "gamma", "normed"],
         lambda t: prog("rms_bwd_colsum", True)([t["g"], t["gamma"], t["normed"]], F, N), 2 * fn + F * 4 + N * 4),
        ("RMSNorm bwd RowSum(g*gamma*normed) (768x8192)", ["g", "gamma", "normed"],
         lambda t: prog("rms_bwd_rowsum", True)([t["g"], t["gamma"], t["normed"]], F, N), 2 * fn + 2 * F * 4),
        ("RMSNorm bwd dx (768x8192)", ["g", "gamma", "mvec", "normed", "rinv"],
         lambda t: prog("rms_bwd_dx")([t["g"], t["gamma"], t["mvec"], t["normed"], t["rinv"]], F, N),
         3 * fn + F * 4 + 2 * N * 4),
        ("SwiGLU bwd grad_gate (3072x8192)", ["gff", "up", "s", "gate"],
         lambda t: prog("swiglu_grad_gate")([t["gff"], t["up"], t["s"], t["gate"], t["s"]], FF, N), 5 * fb),
        ("SwiGLU bwd grad_up (3072x8192)", ["gff", "gate", "s"],
         lambda t: prog("swiglu_grad_up")([t["gff"], t["gate"], t["s"]], FF, N), 4 * fb),
        ("SwiGLU fwd elementwise Mul (3072x8192)", ["gate", "up"],
         lambda t: eng.elementwise_binary("Mul", t["gate"], t["up"]), 3 * fb),
        ("residual Add (768x8192)", ["x", "g"], lambda t: eng.elementwise_binary("Add", t["x"], t["g"]), 3 * fn),
        ("add_inplace (768x8192)", ["normed", "g"], lambda t: eng.add_inplace(t["normed"], t["g"]), 3 * fn),
        ("bias gradient row_reduce_sum (6144x8192)", ["gate2"], lambda t: eng.row_reduce_sum(t["gate2"]),
         2 * fb + 2 * FF * 4),
        ("attention mask Add (98304x1024)", ["scores", "mask"],
         lambda t: eng.elementwise_binary("Add", t["scores"], t["mask"]), 3 * bb),
        ("Softmax fwd rows (98304x1024)", ["scores"], lambda t: prog("softmax_rows")([t["scores"]] * 4, R, C), 2 * bb),
        ("Softmax bwd rows (98304x1024)", ["scores", "sg"],
         lambda t: prog("softmax_rows_backward")([t["scores"], t["sg"], t["scores"], t["sg"]], R, C), 3 * bb),
        ("sparse CE col_softmax_sparse_forward, standalone (32000x8192)", ["logits", "labels"],
         lambda t: eng.col_softmax_sparse_forward(t["logits"], t["labels"], None, V, 1.0 / N),
         2 * V * N * 4 + 2 * N * 4),
        ("gather_rows token embedding (32000x768, 8192 ids)", ["table", "idx"],
         lambda t: eng.gather_rows(t["table"], t["idx"]), 2 * N * F * 4 + N * 4),
        ("transpose (768x8192)", ["x"], lambda t: eng.transpose(t["x"]), 2 * fn),
        ("rearrange_3d (768, 8 x 1024)", ["x"], lambda t: eng.rearrange_3d(t["x"], F, 8, N // 8), 2 * fn),
    ]
    out = []
    for name, inputs, call, nbytes in cases:
        in_bytes = sum(host[k].nbytes for k in set(inputs))
        copies = max(1, min(32, -(-768 * 2 ** 20 // in_bytes)))
        sets = [{k: eng.tensor(host[k]) for k in set(inputs)} for _ in range(copies)]
        it = [0]

        def fn_call():
            t = sets[it[0] % copies]
            it[0] += 1
            return call(t)
        reps = max(20, copies)
        ms = timed_ms(timer, busy, fn_call, reps, steady=False)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out.append({"kernel": name, "bytes": nbytes, "ms": ms, "GB_s": gbs, "frac_of_hbm_peak": gbs / PEAK_HBM_GBS,
                    "input_copies": copies})
        del sets
    eng.sync()
    return out


def pmc_sample(seed):
    """What the rocprofv3 --pmc passes count: one config-4 training step, then a
    256 MiB element-wise copy (Neg: 256 MiB read + 256 MiB written) as the last
    dispatch, the calibration for FETCH_SIZE / WRITE_SIZE."""
    import nnengine
    lib = nnengine.hip_library()
    eng = nnengine.Engine(lib)
    g = init_session(eng, CFG, BATCH, seed)
    loss = g.train_step()
    x = eng.create_tensor(8192, 8192)
    eng.zero(x)
    eng.sync()
    y = eng.elementwise_unary("Neg", x)
    eng.sync()
    del y
    print(json.dumps({"pmc_sample": "1 config-4 train step + 256 MiB Neg copy", "loss": loss}), flush=True)


def host_info(threads):
    """The host the CPU baseline runs on: CPU model and sockets (lscpu), logical CPUs (nproc), the CPUs
    this process may use, and the threads the oracle's pool runs."""
    import subprocess
    info = {"threads": threads, "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            if k.strip() == "Model name":
                info["cpu_model"] = v.strip()
            elif k.strip() == "Socket(s)":
                info["sockets"] = int(v.strip())
    except (OSError, subprocess.SubprocessError, ValueError):
        pass
    return info


def _oracle(threads):
    """The CPU restatement of the reference CpuEngine (oracle/), its pool sized to `threads`."""
    import nnengine
    os.environ["NNORACLE_THREADS"] = str(threads)
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_build", "libnnoracle.so"))
    lib.nnoracle_thread_count.restype = ctypes.c_size_t
    return nnengine.Engine(lib, prefix="nnoracle_"), lib


def _cpu_threads():
    """hardware_concurrency is the reference's pool size (core_threadpool.hpp:612); a GPU box lends one
    GPU's job 16 of its host's CPUs, so the pool is capped at 16 (NNORACLE_THREADS overrides)."""
    return int(os.environ.get("NNORACLE_THREADS", "0")) or min(len(os.sched_getaffinity(0)), 16)


def cpu_leg(seed, steps=3, warmup=1):
    """Config-4 training steps (forward, CE, backward, AdamW) of the oracle at batch 1 of 8, following
    compute_bench's method (src/compute_bench.cpp:36-61): warmup, then timed steps, min and mean."""
    eng, lib = _oracle(_cpu_threads())
    g = init_session(eng, CFG, 1, seed)
    times = []
    for i in range(warmup + steps):
        t0 = time.perf_counter()
        loss = g.train_step()
        dt = time.perf_counter() - t0
        print(f"[bench] cpu baseline {'warmup' if i < warmup else 'timed'} step {dt:.1f}s loss {loss:.4f}",
              file=sys.stderr, flush=True)
        if i >= warmup:
            times.append(dt)
    T = CFG["seq_len"]
    mean, best = sum(times) / len(times), min(times)
    threads = int(lib.nnoracle_thread_count())
    return dict(value=T / mean, unit="tokens/s", cores=threads, kind="port",
                sample=f"config-4 model (12L d768 V32000 T1024 ALiBi) at batch 1 of {BATCH} ({T} tokens): "
                       f"{warmup} warmup + {steps} timed AdamW train steps, mean {mean:.2f} s, min {best:.2f} s; "
                       f"the oracle (CPU restatement of CpuEngine) on {threads} threads",
                tflops=step_flops(CFG, 1) / mean / 1e12, min_s=best, mean_s=mean, host=host_info(threads))


def cpu_legs_other(seed, iters=3, c2_heads=128, c5_heads=12, c5_iters=1):
    """CPU legs of configs 2, 3 and 5 on the oracle, compute_bench's method (src/compute_bench.cpp:36-61):
    one warmup, then timed calls, min and mean. The fused attention primitives are serial loops in the
    reference and in the oracle, so their legs may run on a sample of the heads (c2_heads of config 2's
    128 (batch x head) entries, c5_heads of a config-5 row's 12 heads); each head's work is the same, so
    TFLOP/s carry over and the full call's time is the sample's scaled by the head count. Config 3 runs
    its six GEMMs at full size."""
    eng, lib = _oracle(_cpu_threads())
    rng = np.random.default_rng(seed)
    out = {"host": host_info(int(lib.nnoracle_thread_count()))}

    def bench(fn, n):
        fn()
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return min(ts), sum(ts) / len(ts)

    BH, T, d = c2_heads, 512, 64
    q, k = (eng.tensor(rng.standard_normal((BH * d, T), dtype=np.float32)) for _ in range(2))
    vt = eng.tensor(rng.standard_normal((BH * T, d), dtype=np.float32))
    mask = eng.tensor(eng.build_attention_mask(1, T, 1, False))

    def c2():
        m = eng.batched_matmul_reduce(q, k, BH, "Max", True, False, 0.125, True, mask)
        lsum = eng.batched_matmul_softmax_denom(q, k, m, BH, True, False, 0.125, mask)
        return eng.batched_matmul_softmax_apply(q, k, vt, m, lsum, BH, True, False, 0.125, mask)
    best, mean = bench(c2, iters)
    flop = 4 * d * (T * (T + 1) // 2) * BH
    out["config2_causal_forward"] = {
        "tflops": flop / mean / 1e12, "min_s": best, "mean_s": mean, "full_call_s": mean * 128 / BH,
        "iterations": iters, "warmup": 1,
        "sample": f"{BH} of the 128 (batch x head) entries, T 512, d 64, causal: reduce + denom + apply"}
    print(f"[bench] cpu config 2: {flop / mean / 1e12 * 1e3:.2f} GFLOP/s", file=sys.stderr, flush=True)
    del q, k, vt, mask
    sweep = []
    for name, M, K, N, tA, tB in GEMM_SWEEP[:6]:
        a = eng.tensor(rng.uniform(-1, 1, (M, K)).astype(np.float32))
        b = eng.tensor(rng.uniform(-1, 1, (K, N)).astype(np.float32))
        best, mean = bench(lambda: eng.matmul(a, b), iters)
        fl = 2.0 * M * N * K
        sweep.append({"shape": name, "min_s": best, "mean_s": mean, "gflops": fl / mean / 1e9, "iterations": iters,
                      "warmup": 1})
        print(f"[bench] cpu {name}: {fl / mean / 1e9:.1f} GFLOP/s", file=sys.stderr, flush=True)
    out["config3_gemm"] = sweep
    H, T = c5_heads, 2048
    lens, tot = [], 0
    while tot < T:
        L = min(int(rng.integers(64, 1025)), T - tot)
        lens.append(L)
        tot += L
    ids = np.concatenate([np.full(L, i + 1, dtype=np.uint64) for i, L in enumerate(lens)])
    pairs = sum(L * (L + 1) // 2 for L in lens)
    mk = eng.tensor(eng.build_attention_mask(1, T, 1, False, doc_ids=ids))
    q, k, v, g = (eng.tensor(rng.standard_normal((H * d, T), dtype=np.float32)) for _ in range(4))

    def c5():
        # the GPU leg's call sequence for one packed row (compute_layer.hpp:1196-1221, :1304-1327)
        m = eng.batched_matmul_reduce(q, k, H, "Max", True, False, 0.125, True, mk)
        lsum = eng.batched_matmul_softmax_denom(q, k, m, H, True, False, 0.125, mk)
        vt5 = eng.rearrange_3d(eng.transpose(v), T, H, d)
        o = eng.batched_matmul_softmax_apply(q, k, vt5, m, lsum, H, True, False, 0.125, mk)
        P = eng.batched_matmul(g, v, H, True, False)
        G = eng.rearrange_3d(eng.transpose(g), T, H, d)
        dq, r = eng.batched_matmul_softmax_backward_q(q, k, P, m, lsum, H, True, False, 0.125, mk)
        return o, dq, eng.batched_matmul_softmax_backward_kv(q, k, P, G, r, m, lsum, H, True, False, 0.125, mk)
    best, mean = bench(c5, c5_iters)
    flop = 12 * d * pairs * H
    out["config5_row_forward_backward"] = {
        "tflops": flop / mean / 1e12, "min_s": best, "mean_s": mean, "full_row_s": mean * 12 / H,
        "iterations": c5_iters, "warmup": 1, "allowed_pair_fraction": pairs / (T * T),
        "sample": f"{H} of the 12 heads of one packed row (of 8), T 2048, d 64, documents U{{64..1024}}: "
                  f"forward (reduce, denom, apply) + dP + backward_q + backward_kv"}
    print(f"[bench] cpu config 5: {flop / mean / 1e12 * 1e3:.2f} GFLOP/s", file=sys.stderr, flush=True)
    return out


def cpu_configs_beside_gpu(cpu, attn, sweep):
    """Per-config CPU figures (cpu_legs_other) next to the GPU figures of the same run."""
    out = {"host": cpu["host"]}
    if attn:
        for key, gkey in (("config2_causal_forward", "causal_config2_forward"),
                          ("config5_row_forward_backward", "doc_masked_config5_forward_backward")):
            c, gt = cpu[key], attn[gkey]["tflops"]
            out[key] = dict(c, gpu_tflops=gt, gpu_over_cpu=gt / c["tflops"])
    gpu_by_shape = {r["shape"]: r["tflops"] for r in (sweep or [])}
    out["config3_gemm"] = [dict(r, gpu_gflops=gpu_by_shape[r["shape"]] * 1e3,
                                gpu_over_cpu=gpu_by_shape[r["shape"]] * 1e3 / r["gflops"])
                           if r["shape"] in gpu_by_shape else r for r in cpu["config3_gemm"]]
    return out


def gemm_traffic_bytes():
    """HBM bytes per GEMM launch of the training step, measured by the two
    rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) recorded in
    profiles/gemm_hbm_traffic.txt (key `traffic_bytes_per_launch`); None when
    that measurement is absent."""
    path = os.path.join(ROOT, "profiles", "gemm_hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split("=")[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--skip-cpu-baseline", action="store_true")
    ap.add_argument("--skip-attention", action="store_true")
    ap.add_argument("--skip-inference", action="store_true",
                    help="no incremental-inference leg (kernel traces of the training step alone)")
    ap.add_argument("--skip-gemm-sweep", action="store_true")
    ap.add_argument("--skip-hbm", action="store_true")
    ap.add_argument("--pmc-sample", action="store_true",
                    help="run only the workload the rocprofv3 --pmc passes count (one step + a calibration copy)")
    ap.add_argument("--hbm-only", action="store_true",
                    help="run only the memory-bound kernel leg and print its JSON (for kernel traces)")
    ap.add_argument("--cpu-legs", action="store_true",
                    help="run only the oracle's CPU legs of configs 2, 3 and 5 and print their JSON")
    ap.add_argument("--attention-only", action="store_true",
                    help="run only the attention leg (configs 2 and 5) and print its JSON (for kernel traces)")
    ap.add_argument("--inference-only", action="store_true",
                    help="run only the incremental-inference leg (config-4 model, batch 1) and print its JSON")
    ap.add_argument("--library-gemm", action="store_true",
                    help="time the vendor fp32 GEMM (torch.mm, TF32 off) on the config-4 step's product shapes and "
                         "print its JSON (a comparison, not part of the engine)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    if args.pmc_sample:
        pmc_sample(args.seed)
        return
    if args.attention_only:
        print(json.dumps({"attention": attention_leg(args.seed)}), flush=True)
        return
    if args.library_gemm:
        print(json.dumps({"library_gemm": library_gemm_leg()}), flush=True)
        return
    if args.inference_only:
        import nnengine
        eng = nnengine.Engine(nnengine.hip_library())
        g = init_session(eng, CFG, 1, args.seed)
        print(json.dumps({"inference": inference_leg(g, args.seed)}), flush=True)
        return
    if args.cpu_legs:
        print(json.dumps({"cpu_legs": cpu_legs_other(args.seed)}), flush=True)
        return
    if args.hbm_only:
        print(json.dumps({"hbm_kernels": hbm_leg(args.seed)}), flush=True)
        return
    gpu = gpu_leg(args.steps, args.warmup, args.seed, inference=not args.skip_inference)
    attn = None if args.skip_attention else attention_leg(args.seed)
    sweep = None if args.skip_gemm_sweep else gemm_leg(args.seed)
    hbm = None if args.skip_hbm else hbm_leg(args.seed)
    n_tok = BATCH * CFG["seq_len"]
    ms_per_step = 1000.0 * gpu["elapsed"] / args.steps
    flops = step_flops(CFG, BATCH)
    gemm_avg_ms = gpu["gemm_ms"] / max(gpu["gemm_launches"], 1)
    gemm_flops_per_launch = gpu["gemm_flops"] / max(gpu["gemm_launches"], 1)
    achieved = gpu["gemm_flops"] / (gpu["gemm_ms"] * 1e-3) / 1e12 if gpu["gemm_ms"] > 0 else 0.0
    out = {
        "metric": "GPT 12L/d768 fwd+bwd tokens/s; causal-attn TFLOP/s and % of fp32 MFMA peak",
        "value": n_tok * args.steps / gpu["elapsed"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded tokens U[0,32000), weights N(0,0.02), biases 0, gains 1)",
        "config": {"workload": "BASELINE config 4: GPT train step, 12L d768 12H SwiGLU-3072 RMSNorm ALiBi "
                               "V32000 T1024 B8, AdamW", "global_batch": BATCH, "seq_len": CFG["seq_len"],
                   "parallelism": "none (1 GPU)"},
        "model_tflops": flops / (ms_per_step * 1e-3) / 1e12,
        "step_tflop": flops / 1e12,
        "roofline": {"bound": "mfma", "kernel": "fp32 MFMA GEMM (all matmul/batched_matmul launches)",
                     "achieved": achieved, "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_FP32_MFMA_TFLOPS, "traffic": gemm_traffic_bytes(),
                     "launches": gpu["gemm_launches"], "avg_launch_ms": gemm_avg_ms,
                     "flop_per_launch": gemm_flops_per_launch,
                     "share_of_step": gpu["gemm_ms"] / (gpu["elapsed"] * 1000.0),
                     "by_shape": gpu["gemm_shapes"]},
    }
    out["inference"] = gpu["inference"]
    if attn is not None:
        out["attention"] = attn
    if sweep is not None:
        out["gemm_sweep_config3"] = sweep
    if hbm is not None:
        out["hbm_kernels"] = hbm
    if not args.skip_cpu_baseline:
        cpu = cpu_leg(args.seed)
        out["cpu_baseline"] = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample", "tflops", "min_s",
                                                   "mean_s", "host")}
        # configs 2, 3 and 5 on the same host in the same run, bounded samples (about 20 s)
        others = cpu_legs_other(args.seed, iters=3, c2_heads=16, c5_heads=2, c5_iters=1)
        out["cpu_baseline"]["configs"] = cpu_configs_beside_gpu(others, attn, sweep)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

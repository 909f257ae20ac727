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
fraction of the fp32 MFMA peak, timed with HIP events on the engine's stream.
`cpu_baseline` runs the CPU restatement of the reference CpuEngine (oracle/,
loaded only for this leg) on a bounded sample of the same workload: one full
training step at batch 1 of 8.
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


def gpu_leg(steps, warmup, seed):
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
    launches, flops, ms = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    eng._check(lib.nnhip_engine_profile_gemm_read(eng._e, ctypes.byref(launches), ctypes.byref(flops),
                                                  ctypes.byref(ms)))
    eng._check(lib.nnhip_engine_profile_gemm(eng._e, 0))
    print(f"[bench] timed {steps} steps in {elapsed:.3f}s, losses {[round(x, 4) for x in losses]}",
          file=sys.stderr, flush=True)
    for x in losses:
        if not math.isfinite(x):
            raise RuntimeError(f"non-finite loss {x}")
    return dict(elapsed=elapsed, gemm_launches=launches.value, gemm_flops=flops.value, gemm_ms=ms.value,
                losses=losses)


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


def attention_leg(seed, reps=5):
    """BASELINE configs 2 and 5 through the engine's fused attention primitives."""
    import nnengine
    lib = nnengine.hip_library()
    eng = nnengine.Engine(lib)
    timer = StreamTimer(lib, eng)
    rng = np.random.default_rng(seed)
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
    fwd()
    timer.start()
    for _ in range(reps):
        fwd()
    ms = timer.stop_ms() / reps
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

    def fwd_bwd():
        for q, k, v, g, mk in rows:
            m = eng.batched_matmul_reduce(q, k, H, "Max", True, False, 0.125, True, mk)
            l = eng.batched_matmul_softmax_denom(q, k, m, H, True, False, 0.125, mk)
            vt = eng.rearrange_3d(eng.transpose(v), T, H, d)
            eng.batched_matmul_softmax_apply(q, k, vt, m, l, H, True, False, 0.125, mk)
            P = eng.batched_matmul(g, v, H, True, False)
            G = eng.rearrange_3d(eng.transpose(g), T, H, d)
            dq, r = eng.batched_matmul_softmax_backward_q(q, k, P, m, l, H, True, False, 0.125, mk)
            eng.batched_matmul_softmax_backward_kv(q, k, P, G, r, m, l, H, True, False, 0.125, mk)
    fwd_bwd()
    timer.start()
    for _ in range(reps):
        fwd_bwd()
    ms = timer.stop_ms() / reps
    flop = 12 * d * pairs * H
    out["doc_masked_config5_forward_backward"] = {
        "tflops": flop / (ms * 1e-3) / 1e12, "frac_of_fp32_mfma_peak": flop / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
        "ms": ms, "flop": flop, "allowed_pair_fraction": pairs / (B * T * T),
        "workload": "B8 x H12, T2048, d64, doc lengths U{64..1024}: forward (reduce, denom, apply) + dP GEMM + "
                    "backward_q + backward_kv, all 8 rows"}
    eng.sync()
    return out


def cpu_leg(seed):
    import nnengine
    threads = int(os.environ.get("NNORACLE_THREADS", "0")) or min(os.cpu_count() or 1, 16)
    os.environ["NNORACLE_THREADS"] = str(threads)
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_build", "libnnoracle.so"))
    eng = nnengine.Engine(lib, prefix="nnoracle_")
    lib.nnoracle_thread_count.restype = ctypes.c_size_t
    g = init_session(eng, CFG, 1, seed)
    t0 = time.perf_counter()
    loss = g.train_step()
    dt = time.perf_counter() - t0
    print(f"[bench] cpu baseline step {dt:.1f}s loss {loss:.4f}", file=sys.stderr, flush=True)
    T = CFG["seq_len"]
    return dict(value=T / dt, unit="tokens/s", cores=int(lib.nnoracle_thread_count()), kind="port",
                sample=f"1 AdamW train step of the config-4 model on batch 1 of {BATCH} ({T} tokens), "
                       f"{dt:.1f} s", seconds=dt)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--skip-cpu-baseline", action="store_true")
    ap.add_argument("--skip-attention", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    gpu = gpu_leg(args.steps, args.warmup, args.seed)
    attn = None if args.skip_attention else attention_leg(args.seed)
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
                     "frac": achieved / PEAK_FP32_MFMA_TFLOPS, "traffic": None,
                     "launches": gpu["gemm_launches"], "avg_launch_ms": gemm_avg_ms,
                     "flop_per_launch": gemm_flops_per_launch,
                     "share_of_step": gpu["gemm_ms"] / (gpu["elapsed"] * 1000.0)},
    }
    if attn is not None:
        out["attention"] = attn
    if not args.skip_cpu_baseline:
        cpu = cpu_leg(args.seed)
        out["cpu_baseline"] = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

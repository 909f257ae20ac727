"""nnengine — Python host binding of the HIP compute engine's C-ABI.

Mirrors the reference's nn::ComputeEngine operator interface
(/root/reference/include/neuralnet.cpp/compute_engine.hpp:87-410): the same
primitive names, argument meaning and error behaviour (a failing primitive
raises EngineError carrying the engine's message, the way the reference
returns std::unexpected(Error{...})). Tensors are row-major float32 handles
owned by the engine; index tensors hold integers as floats.

The binding is generic over the symbol prefix of include/nnhip_engine.h so
that the same Python code drives any library exporting that ABI. The
product library is libnnhip.so (``hip_library()``), which fails loudly when
it has not been built: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIB_PATH = os.path.join(HERE, "lib", "libnnhip.so")

# Op codes of include/nnhip_engine.h (enum nnhip_op).
OP = dict(CLONE=1, SLICE_ROWS=2, INSERT_ROWS=3, GATHER_ROWS=4, SCATTER_ADD_ROWS=5, REARRANGE_3D=6,
          TRANSPOSE=7, MATMUL=8, BATCHED_MATMUL=9, BMM_REDUCE=10, BMM_DENOM=11, BMM_APPLY=12, BMM_BWD_Q=13,
          BMM_BWD_KV=14, COL_SOFTMAX_DENOM=15, COL_SOFTMAX_SPARSE=16, ADD_INPLACE=17, SCALE_INPLACE=18,
          AXPY_INPLACE=19, ZERO=20, ROW_REDUCE_SUM=21, COL_REDUCE_SUM=22, ROW_REDUCE_MAX=23,
          COL_REDUCE_MAX=24, BROADCAST_ROW=25, BROADCAST_COL=26, UNARY=27, BINARY=28, BINARY_SCALAR=29,
          SELECT_SCALAR_COND=30)

# Enum values of compute_engine.hpp:43-82.
UNARY = dict(Neg=0, Exp=1, Log=2, Sqrt=3, Rsqrt=4, Abs=5, Tanh=6)
BINARY = dict(Add=0, Sub=1, Mul=2, Div=3, Max=4, Min=5)
COMPARE = dict(Lt=0, Le=1, Gt=2, Ge=3, Eq=4, Ne=5)
REDUCE = dict(Sum=0, Max=1, Min=2)
POS_ENC = dict(learned=0, sinusoidal=1, alibi=2, rope=3)


class EngineError(RuntimeError):
    pass


def hip_library() -> ctypes.CDLL:
    """Load the product library. Raises if it has not been built."""
    if not os.path.exists(HIP_LIB_PATH):
        raise EngineError(f"{HIP_LIB_PATH} is missing: run __graft_entry__.build() first "
                          "(there is no CPU fallback)")
    return ctypes.CDLL(HIP_LIB_PATH)


def create_engine(use_hip: bool = False, use_cuda: bool = False, use_gpu: bool = False,
                  verbose: bool = False) -> "Engine":
    """cli::create_engine with the reference's selection rules (cli/engine_factory.hpp:45-88) plus use_hip:
    the requested engine or EngineError, never a fallback to another engine."""
    lib = hip_library()
    fn = lib.nnhip_engine_select
    fn.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_void_p)]
    h = ctypes.c_void_p()
    if fn(int(use_hip), int(use_cuda), int(use_gpu), int(verbose), ctypes.byref(h)) != 0:
        lib.nnhip_last_error.restype = ctypes.c_char_p
        raise EngineError(lib.nnhip_last_error().decode())
    return Engine(lib, handle=h.value)


class _GptConfig(ctypes.Structure):
    _fields_ = [("vocab_size", ctypes.c_size_t), ("d_model", ctypes.c_size_t), ("seq_len", ctypes.c_size_t),
                ("num_heads", ctypes.c_size_t), ("d_ff", ctypes.c_size_t), ("num_layers", ctypes.c_size_t),
                ("pos_enc", ctypes.c_uint32), ("lr", ctypes.c_float), ("beta1", ctypes.c_float),
                ("beta2", ctypes.c_float), ("eps", ctypes.c_float), ("weight_decay", ctypes.c_float),
                ("activation", ctypes.c_uint32), ("norm_type", ctypes.c_uint32), ("optimizer", ctypes.c_uint32)]


ACTIVATION = dict(gelu=0, swiglu=1)
NORM = dict(layernorm=0, rmsnorm=1)
OPTIMIZER = dict(adamw=0, adam=1, sgd=2, sgd_momentum=3, muon=4)


def _bind(lib: ctypes.CDLL, prefix: str):
    vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    fp = ctypes.POINTER(ctypes.c_float)
    u64p = ctypes.POINTER(ctypes.c_uint64)
    sig = {
        "last_error": (ctypes.c_char_p, []),
        "engine_create": (i32, [ctypes.POINTER(vp)]),
        "engine_destroy": (None, [vp]),
        "engine_sync": (i32, [vp]),
        "tensor_create": (vp, [vp, sz, sz]),
        "tensor_from_host": (vp, [vp, fp, sz, sz]),
        "tensor_to_host": (i32, [vp, vp, fp]),
        "tensor_copy_from_host": (i32, [vp, vp, fp]),
        "tensor_rows": (sz, [vp]),
        "tensor_cols": (sz, [vp]),
        "tensor_data_ptr": (vp, [vp]),
        "tensor_release": (None, [vp]),
        "engine_op": (i32, [vp, i32, ctypes.POINTER(vp), sz, ctypes.POINTER(vp), sz,
                            ctypes.POINTER(ctypes.c_double), sz]),
        "engine_eval_expr": (i32, [vp, ctypes.POINTER(ctypes.c_uint8), sz, ctypes.POINTER(ctypes.c_uint8),
                                   ctypes.POINTER(ctypes.c_uint32), sz, fp, sz, ctypes.c_uint32,
                                   ctypes.POINTER(vp), sz, sz, sz, i32, ctypes.POINTER(vp)]),
        "gpt_create": (i32, [vp, ctypes.POINTER(_GptConfig), ctypes.POINTER(vp)]),
        "gpt_destroy": (None, [vp]),
        "gpt_num_params": (sz, [vp]),
        "gpt_param_shape": (i32, [vp, sz, ctypes.POINTER(sz), ctypes.POINTER(sz)]),
        "gpt_set_param": (i32, [vp, sz, fp]),
        "gpt_get_param": (i32, [vp, sz, fp]),
        "gpt_get_grad": (i32, [vp, sz, fp]),
        "gpt_set_doc_ids": (i32, [vp, ctypes.POINTER(ctypes.c_uint64), sz]),
        "gpt_load_batch": (i32, [vp, fp, sz, sz, ctypes.POINTER(ctypes.c_uint64), fp]),
        "gpt_forward_loss": (i32, [vp, fp]),
        "gpt_logits": (i32, [vp, fp]),
        "gpt_backward": (i32, [vp]),
        "gpt_optimizer_step": (i32, [vp]),
        "gpt_zero_grad": (i32, [vp]),
        "gpt_train_step": (i32, [vp, fp]),
        "gpt_backward_scaled": (i32, [vp, ctypes.c_float]),
        "gpt_save": (i32, [vp, ctypes.c_char_p, ctypes.c_char_p, sz]),
        "gpt_load": (i32, [vp, ctypes.c_char_p, ctypes.c_char_p, sz, ctypes.POINTER(ctypes.c_size_t)]),
        "window_batch": (i32, [u64p, u64p, sz, u64p, sz, sz, ctypes.c_uint64, fp, u64p, fp, u64p,
                               ctypes.POINTER(ctypes.c_size_t)]),
        "gpt_clip_grad_norm": (i32, [vp, ctypes.c_float]),
        "gpt_train_step_ex": (i32, [vp, ctypes.c_size_t, ctypes.c_float, ctypes.c_int, fp]),
        "gpt_forward_step": (i32, [vp, ctypes.c_uint64, sz, sz, fp]),
        "gpt_reset_cache": (i32, [vp]),
        "gpt_generate": (i32, [vp, u64p, sz, sz, ctypes.c_float, ctypes.c_uint64, sz, ctypes.c_uint64, u64p, sz,
                               ctypes.POINTER(ctypes.c_size_t)]),
        "build_attention_mask": (i32, [sz, sz, sz, i32, fp, ctypes.POINTER(ctypes.c_uint64), sz, fp]),
    }
    fns = {}
    for name, (res, args) in sig.items():
        f = getattr(lib, prefix + name)
        f.restype = res
        f.argtypes = args
        fns[name] = f
    return fns


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Tensor:
    """Engine-owned (rows, cols) float32 tensor handle."""

    def __init__(self, eng: "Engine", handle: int):
        self._eng = eng
        self._h = ctypes.c_void_p(handle)

    @property
    def rows(self) -> int:
        return self._eng._f["tensor_rows"](self._h)

    @property
    def cols(self) -> int:
        return self._eng._f["tensor_cols"](self._h)

    @property
    def shape(self):
        return (self.rows, self.cols)

    def data_ptr(self) -> int:
        return self._eng._f["tensor_data_ptr"](self._h) or 0

    def device_ptr(self) -> int:
        """The pointer for a raw reader: everything the values depend on is queued first
        (nnhip_tensor_device_ptr); the memory holds them once the engine's stream gets there."""
        f = getattr(self._eng._lib, self._eng._prefix + "tensor_device_ptr")
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
        out = ctypes.c_void_p()
        self._eng._check(f(self._eng._e, self._h, ctypes.byref(out)))
        return out.value or 0

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=np.float32)
        self._eng._check(self._eng._f["tensor_to_host"](self._eng._e, self._h, _fptr(out)))
        return out

    def copy_from(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=np.float32)
        self._eng._check(self._eng._f["tensor_copy_from_host"](self._eng._e, self._h, _fptr(a)))

    def __del__(self):
        try:
            if self._h:
                self._eng._f["tensor_release"](self._h)
                self._h = None
        except Exception:
            pass


class Engine:
    """Python mirror of nn::ComputeEngine over a library exporting include/nnhip_engine.h."""

    def __init__(self, lib: Optional[ctypes.CDLL] = None, prefix: str = "nnhip_", handle: Optional[int] = None):
        self._lib = lib if lib is not None else hip_library()
        self._prefix = prefix
        self._f = _bind(self._lib, prefix)
        if handle is not None:   # an engine already created (create_engine)
            self._e = ctypes.c_void_p(handle)
            return
        e = ctypes.c_void_p()
        self._check(self._f["engine_create"](ctypes.byref(e)))
        self._e = e

    # -- plumbing -------------------------------------------------------------
    def _err(self) -> str:
        m = self._f["last_error"]()
        return m.decode() if m else "unknown error"

    def _check(self, rc: int) -> None:
        if rc != 0:
            raise EngineError(self._err())

    def close(self) -> None:
        if getattr(self, "_e", None):
            self._f["engine_destroy"](self._e)
            self._e = None

    def sync(self) -> None:
        self._check(self._f["engine_sync"](self._e))

    def settle(self) -> None:
        """Launches deferred attention work still referenced, without waiting (HIP engine only)."""
        fn = getattr(self._lib, "nnhip_engine_settle", None)
        if fn is not None:
            fn.argtypes = [ctypes.c_void_p]
            self._check(fn(self._e))

    def set_score_budget(self, nbytes: int) -> None:
        """Bytes of attention score blocks the two-pass chain may keep from forward to backward
        (HIP engine only; 0: every backward forms its scores again)."""
        fn = self._lib.nnhip_engine_set_score_budget
        fn.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        self._check(fn(self._e, nbytes))

    def tensor(self, a) -> Tensor:
        a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
        if a.ndim == 1:
            a = a.reshape(1, -1)
        h = self._f["tensor_from_host"](self._e, _fptr(a), a.shape[0], a.shape[1])
        if not h:
            raise EngineError(self._err())
        return Tensor(self, h)

    def create_tensor(self, rows: int, cols: int) -> Tensor:
        return Tensor(self, self._f["tensor_create"](self._e, rows, cols))

    def _op(self, op: str, ins: Sequence[Tensor], n_out: int, args: Sequence[float] = ()) -> List[Tensor]:
        inh = (ctypes.c_void_p * max(1, len(ins)))(*[t._h.value for t in ins])
        outh = (ctypes.c_void_p * max(1, n_out))()
        arr = (ctypes.c_double * max(1, len(args)))(*[float(x) for x in args])
        self._check(self._f["engine_op"](self._e, OP[op], inh, len(ins), outh, n_out, arr, len(args)))
        return [Tensor(self, outh[i]) for i in range(n_out)]

    # -- ComputeEngine primitives (names as in compute_engine.hpp) -------------
    def clone(self, A): return self._op("CLONE", [A], 1)[0]
    def slice_rows(self, A, start, count): return self._op("SLICE_ROWS", [A], 1, [start, count])[0]
    def insert_rows(self, dst, start, src): self._op("INSERT_ROWS", [dst, src], 0, [start])
    def gather_rows(self, table, idx): return self._op("GATHER_ROWS", [table, idx], 1)[0]
    def scatter_add_rows(self, dst, idx, grad): self._op("SCATTER_ADD_ROWS", [dst, idx, grad], 0)

    def rearrange_3d(self, X, M, B, N, inverse=False):
        return self._op("REARRANGE_3D", [X], 1, [M, B, N, inverse])[0]

    def transpose(self, A): return self._op("TRANSPOSE", [A], 1)[0]

    def matmul(self, A, B, transA=False, transB=False):
        return self._op("MATMUL", [A, B], 1, [transA, transB])[0]

    def batched_matmul(self, A, B, batch, transA=False, transB=False, alpha=1.0):
        return self._op("BATCHED_MATMUL", [A, B], 1, [batch, transA, transB, alpha])[0]

    def batched_matmul_reduce(self, A, B, batch, op, transA, transB, alpha, reduce_cols=True, mask=None):
        ins = [A, B] + ([mask] if mask is not None else [])
        return self._op("BMM_REDUCE", ins, 1, [batch, REDUCE[op] if isinstance(op, str) else op, transA, transB,
                                               alpha, reduce_cols])[0]

    def batched_matmul_softmax_denom(self, A, B, row_max, batch, transA, transB, alpha, mask=None):
        ins = [A, B, row_max] + ([mask] if mask is not None else [])
        return self._op("BMM_DENOM", ins, 1, [batch, transA, transB, alpha])[0]

    def batched_matmul_softmax_apply(self, A, B, V, row_max, denom, batch, transA, transB, alpha, mask=None):
        ins = [A, B, V, row_max, denom] + ([mask] if mask is not None else [])
        return self._op("BMM_APPLY", ins, 1, [batch, transA, transB, alpha])[0]

    def batched_matmul_softmax_backward_q(self, A, B, P, row_max, denom, batch, transA, transB, alpha, mask=None):
        """Returns (grad_Q, R)."""
        ins = [A, B, P, row_max, denom] + ([mask] if mask is not None else [])
        dq, r = self._op("BMM_BWD_Q", ins, 2, [batch, transA, transB, alpha])
        return dq, r

    def batched_matmul_softmax_backward_kv(self, A, B, P, G, R, row_max, denom, batch, transA, transB, alpha,
                                           mask=None):
        """Returns (grad_K, grad_V)."""
        ins = [A, B, P, G, R, row_max, denom] + ([mask] if mask is not None else [])
        dk, dv = self._op("BMM_BWD_KV", ins, 2, [batch, transA, transB, alpha])
        return dk, dv

    def col_softmax_denom(self, logits, col_max):
        return self._op("COL_SOFTMAX_DENOM", [logits, col_max], 1)[0]

    def col_softmax_sparse_forward(self, logits, labels, mask, vocab_size, inv_num_valid):
        """Returns (grad, loss_vec)."""
        ins = [logits, labels] + ([mask] if mask is not None else [])
        g, lv = self._op("COL_SOFTMAX_SPARSE", ins, 2, [vocab_size, inv_num_valid])
        return g, lv

    def add_inplace(self, A, B): self._op("ADD_INPLACE", [A, B], 0)
    def scale_inplace(self, A, s): self._op("SCALE_INPLACE", [A], 0, [s])
    def axpy_inplace(self, A, s, B): self._op("AXPY_INPLACE", [A, B], 0, [s])
    def zero(self, A): self._op("ZERO", [A], 0)
    def row_reduce_sum(self, A): return self._op("ROW_REDUCE_SUM", [A], 1)[0]
    def col_reduce_sum(self, A): return self._op("COL_REDUCE_SUM", [A], 1)[0]
    def row_reduce_max(self, A): return self._op("ROW_REDUCE_MAX", [A], 1)[0]
    def col_reduce_max(self, A): return self._op("COL_REDUCE_MAX", [A], 1)[0]
    def broadcast_row_inplace(self, A, v, op): self._op("BROADCAST_ROW", [A, v], 0, [BINARY[op]])
    def broadcast_col_inplace(self, A, v, op): self._op("BROADCAST_COL", [A, v], 0, [BINARY[op]])
    def elementwise_unary(self, op, A): return self._op("UNARY", [A], 1, [UNARY[op]])[0]
    def elementwise_binary(self, op, A, B): return self._op("BINARY", [A, B], 1, [BINARY[op]])[0]

    def elementwise_binary_scalar(self, op, A, s, scalar_first=False):
        return self._op("BINARY_SCALAR", [A], 1, [BINARY[op], s, scalar_first])[0]

    def elementwise_select_scalar_cond(self, cmp, A, scalar_b, then_t, scalar_else):
        return self._op("SELECT_SCALAR_COND", [A, then_t], 1, [COMPARE[cmp], scalar_b, scalar_else])[0]

    def eval_expr(self, spec: "ExprSpec", inputs: Sequence[Tensor], rows: int, cols: int, vector_out=False):
        ins, vk, vp, cs = spec.serialise()
        inh = (ctypes.c_void_p * max(1, len(inputs)))(*[t._h.value for t in inputs])
        out = ctypes.c_void_p()
        self._check(self._f["engine_eval_expr"](
            self._e, ins.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), len(spec.instrs),
            vk.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), vp.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
            len(spec.views), _fptr(cs), len(spec.consts), spec.num_regs, inh, len(inputs), rows, cols,
            1 if vector_out else 0, ctypes.byref(out)))
        return Tensor(self, out.value)

    def eval_expr_reduce(self, spec, inputs, rows, cols):
        return self.eval_expr(spec, inputs, rows, cols, vector_out=True)

    # -- pure host helpers ------------------------------------------------------
    def build_attention_mask(self, batch, seq, heads, use_alibi, slopes=(), doc_ids=()):
        if use_alibi and len(slopes) != heads:
            raise EngineError(f"build_attention_mask: ALiBi needs one slope per head ({heads}), got {len(slopes)}")
        sl = np.asarray(list(slopes) if len(slopes) else [0.0], dtype=np.float32)
        di = np.asarray(list(doc_ids) if len(doc_ids) else [0], dtype=np.uint64)
        out = np.empty((batch * heads * seq, seq), dtype=np.float32)
        self._check(self._f["build_attention_mask"](batch, seq, heads, 1 if use_alibi else 0, _fptr(sl),
                                                    di.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                                    len(doc_ids), _fptr(out)))
        return out

    def window_batch(self, flow, starts, seq, pad_id, flow_doc=None):
        """One training batch cut from a token flow (src/text_train.cpp:1137-1172): returns
        tokens (seq, batch) float32, labels and loss_mask (batch*seq,), doc_ids (batch*seq,) or
        None, and the number of positions in the loss."""
        u64 = ctypes.POINTER(ctypes.c_uint64)
        fl = np.ascontiguousarray(np.asarray(flow, dtype=np.uint64))
        st = np.ascontiguousarray(np.asarray(starts, dtype=np.uint64))
        fd = None if flow_doc is None else np.ascontiguousarray(np.asarray(flow_doc, dtype=np.uint64))
        batch = st.size
        tokens = np.empty((seq, batch), dtype=np.float32)
        labels = np.empty(batch * seq, dtype=np.uint64)
        mask = np.empty(batch * seq, dtype=np.float32)
        docs = None if fd is None else np.empty(batch * seq, dtype=np.uint64)
        valid = ctypes.c_size_t()
        self._check(self._f["window_batch"](fl.ctypes.data_as(u64), None if fd is None else fd.ctypes.data_as(u64),
                                            fl.size, st.ctypes.data_as(u64), batch, seq, int(pad_id), _fptr(tokens),
                                            labels.ctypes.data_as(u64), _fptr(mask),
                                            None if docs is None else docs.ctypes.data_as(u64), ctypes.byref(valid)))
        return tokens, labels, mask, docs, valid.value

    def gpt(self, **cfg) -> "GptSession":
        return GptSession(self, **cfg)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def layer_program(lib: ctypes.CDLL, name: str, param: int = 0, prefix: str = "nnhip_") -> dict:
    """A program of include/nn/layer_exprs.hpp as the library builds it (nnhip_layer_program):
    instrs (8-tuples), views ((kind, negate, param)), consts, num_regs and slot_args (the C++
    builder's argument each input slot reads)."""
    fn = getattr(lib, prefix + "layer_program")
    sz = ctypes.POINTER(ctypes.c_size_t)
    fn.argtypes = [ctypes.c_char_p, ctypes.c_uint32, ctypes.c_void_p, sz, ctypes.c_void_p, ctypes.c_void_p, sz,
                   ctypes.c_void_p, sz, ctypes.POINTER(ctypes.c_uint32), ctypes.c_void_p, sz]
    ins = np.zeros((64, 8), np.uint8)
    vk, vp = np.zeros(16, np.uint8), np.zeros(8, np.uint32)
    cs, sa = np.zeros(16, np.float32), np.zeros(8, np.int32)
    ni, nv, nc, ns = (ctypes.c_size_t() for _ in range(4))
    nr = ctypes.c_uint32()
    rc = fn(name.encode(), param, ins.ctypes.data, ctypes.byref(ni), vk.ctypes.data, vp.ctypes.data,
            ctypes.byref(nv), cs.ctypes.data, ctypes.byref(nc), ctypes.byref(nr), sa.ctypes.data, ctypes.byref(ns))
    if rc != 0:
        err = getattr(lib, prefix + "last_error")
        err.restype = ctypes.c_char_p
        raise EngineError(err().decode())
    return dict(instrs=[tuple(int(x) for x in r) for r in ins[:ni.value]],
                views=[(int(vk[2 * i]), int(vk[2 * i + 1]), int(vp[i])) for i in range(nv.value)],
                consts=[float(c) for c in cs[:nc.value]], num_regs=int(nr.value),
                slot_args=[int(x) for x in sa[:ns.value]])


# ExprSpec codes (expr_spec.hpp:30-62, 94-101, 116-159).
EXPR_OP = dict(Neg=0, Exp=1, Log=2, Sqrt=3, Rsqrt=4, Abs=5, Tanh=6, Add=7, Sub=8, Mul=9, Div=10, Max=11, Min=12,
               Lt=13, Le=14, Gt=15, Ge=16, Eq=17, Ne=18, Select=19, ColSum=20, ColMax=21, RowSum=22, RowMax=23)
OPND = dict(Reg=0, Input=1, Const=2, Fanout=3, Reduce=4)
VIEW = dict(Linear=0, RotateHalf=1, RowMod=2, ColReduceSum=3, ColReduceMax=4, RowReduceSum=5, RowReduceMax=6,
            RowBroadcast=7, ColBroadcast=8)


@dataclass
class ExprSpec:
    """Serialisable ExprSpec: instrs are 8-tuples (op,dst,a.kind,a.idx,b.kind,b.idx,c.kind,c.idx),
    views are (kind, negate_first_half, param)."""
    instrs: list = field(default_factory=list)
    views: list = field(default_factory=list)
    consts: list = field(default_factory=list)
    num_regs: int = 0

    def ins(self, op, a=(0, 0), b=(0, 0), c=(0, 0), dst=None):
        d = self.num_regs if dst is None else dst
        if dst is None:
            self.num_regs += 1
        self.instrs.append((EXPR_OP[op], d, a[0], a[1], b[0], b[1], c[0], c[1]))
        return d

    def view(self, kind, param=0, negate=0):
        self.views.append((VIEW[kind], negate, param))
        return len(self.views) - 1

    def const(self, v):
        self.consts.append(float(v))
        return len(self.consts) - 1

    def serialise(self):
        """Arrays in the layout of nnhip_engine_eval_expr: instrs (n,8) u8, view kinds
        {kind, negate} pairs u8, view params u32, consts f32 (each at least one entry long)."""
        ins = np.zeros((max(1, len(self.instrs)), 8), dtype=np.uint8)
        for i, t in enumerate(self.instrs):
            ins[i] = t
        vk = np.zeros(max(1, 2 * len(self.views)), dtype=np.uint8)
        vp = np.zeros(max(1, len(self.views)), dtype=np.uint32)
        for i, (k, neg, p) in enumerate(self.views):
            vk[2 * i], vk[2 * i + 1], vp[i] = k, neg, p
        cs = np.asarray(self.consts if self.consts else [0.0], dtype=np.float32)
        return ins, vk, vp, cs


def reg(i): return (OPND["Reg"], i)
def inp(i): return (OPND["Input"], i)
def cst(i): return (OPND["Const"], i)
def red(i): return (OPND["Reduce"], i)


class GptSession:
    """GPTModel + sparse cross-entropy + AdamW on one engine (include/nnhip_engine.h)."""

    def __init__(self, eng: Engine, vocab_size, d_model, seq_len, num_heads, d_ff, num_layers, pos_enc="learned",
                 lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, activation="swiglu", norm="rmsnorm",
                 optimizer="adamw"):
        self._eng = eng
        self._f = eng._f
        cfg = _GptConfig(vocab_size, d_model, seq_len, num_heads, d_ff, num_layers, POS_ENC[pos_enc], lr, beta1,
                         beta2, eps, weight_decay, ACTIVATION[activation], NORM[norm], OPTIMIZER[optimizer])
        g = ctypes.c_void_p()
        eng._check(self._f["gpt_create"](eng._e, ctypes.byref(cfg), ctypes.byref(g)))
        self._g = g
        self.vocab_size = vocab_size

    def num_params(self) -> int:
        return self._f["gpt_num_params"](self._g)

    def param_shapes(self):
        out = []
        for i in range(self.num_params()):
            r, c = ctypes.c_size_t(), ctypes.c_size_t()
            self._eng._check(self._f["gpt_param_shape"](self._g, i, ctypes.byref(r), ctypes.byref(c)))
            out.append((r.value, c.value))
        return out

    def set_params(self, arrays) -> None:
        for i, a in enumerate(arrays):
            a = np.ascontiguousarray(a, dtype=np.float32)
            self._eng._check(self._f["gpt_set_param"](self._g, i, _fptr(a)))

    def _read(self, fn, i, shape):
        out = np.empty(shape, dtype=np.float32)
        self._eng._check(self._f[fn](self._g, i, _fptr(out)))
        return out

    def params(self):
        return [self._read("gpt_get_param", i, s) for i, s in enumerate(self.param_shapes())]

    def grads(self):
        return [self._read("gpt_get_grad", i, s) for i, s in enumerate(self.param_shapes())]

    def set_doc_ids(self, ids) -> None:
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.uint64).reshape(-1))
        self._eng._check(self._f["gpt_set_doc_ids"](self._g, a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                                    a.size))

    def load_batch(self, tokens: np.ndarray, labels: np.ndarray, loss_mask: Optional[np.ndarray] = None) -> None:
        """tokens (seq, batch) ids; labels (batch*seq,) batch-major."""
        tk = np.ascontiguousarray(tokens, dtype=np.float32)
        lb = np.ascontiguousarray(np.asarray(labels, dtype=np.uint64).reshape(-1))
        self._n = tk.size
        mk = None if loss_mask is None else np.ascontiguousarray(loss_mask, dtype=np.float32)
        self._eng._check(self._f["gpt_load_batch"](self._g, _fptr(tk), tk.shape[0], tk.shape[1],
                                                   lb.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                                   _fptr(mk) if mk is not None else None))

    def forward_loss(self) -> float:
        v = ctypes.c_float()
        self._eng._check(self._f["gpt_forward_loss"](self._g, ctypes.byref(v)))
        return v.value

    def logits(self) -> np.ndarray:
        out = np.empty((self.vocab_size, self._n), dtype=np.float32)
        self._eng._check(self._f["gpt_logits"](self._g, _fptr(out)))
        return out

    def backward(self) -> None:
        self._eng._check(self._f["gpt_backward"](self._g))

    def optimizer_step(self) -> None:
        self._eng._check(self._f["gpt_optimizer_step"](self._g))

    def zero_grad(self) -> None:
        self._eng._check(self._f["gpt_zero_grad"](self._g))

    def train_step(self) -> float:
        v = ctypes.c_float()
        self._eng._check(self._f["gpt_train_step"](self._g, ctypes.byref(v)))
        return v.value

    def save(self, path: str, tokenizer: bytes = b"") -> None:
        """The reference's model file, format v4 (model_serialization.hpp:380-425)."""
        self._eng._check(self._f["gpt_save"](self._g, path.encode(), tokenizer or None, len(tokenizer)))

    def load(self, path: str) -> bytes:
        """Loads parameters from a format-v4 model file whose spec matches this session's model
        (the AdamW state starts afresh); returns the embedded tokenizer bytes. One call: the
        tokenizer buffer is sized by the file, which holds it."""
        n = ctypes.c_size_t()
        buf = ctypes.create_string_buffer(max(1, os.path.getsize(path)))
        self._eng._check(self._f["gpt_load"](self._g, path.encode(), buf, len(buf), ctypes.byref(n)))
        return buf.raw[:n.value]

    def forward_step(self, token: int, pos: int, cur_len: int) -> np.ndarray:
        """GPTModel::forward_step with the session's KV caches: logits (vocab,) of one token."""
        out = np.empty(self.vocab_size, dtype=np.float32)
        self._eng._check(self._f["gpt_forward_step"](self._g, int(token), int(pos), int(cur_len), _fptr(out)))
        return out

    def reset_cache(self) -> None:
        self._eng._check(self._f["gpt_reset_cache"](self._g))

    def generate(self, prompt, max_new: int, temperature: float = 0.0, eos: int = 2 ** 64 - 1, min_new: int = 0,
                 seed: int = 0):
        """GPTModel::generate (sampling with KV caches); the generated token ids."""
        pr = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint64))
        out = np.zeros(max(1, max_new), dtype=np.uint64)
        n = ctypes.c_size_t()
        u64p = ctypes.POINTER(ctypes.c_uint64)
        self._eng._check(self._f["gpt_generate"](self._g, pr.ctypes.data_as(u64p), pr.size, int(max_new),
                                                 float(temperature), int(eos), int(min_new), int(seed),
                                                 out.ctypes.data_as(u64p), out.size, ctypes.byref(n)))
        return out[:n.value].astype(np.int64).tolist()

    def backward_scaled(self, grad_scale: float) -> None:
        """Backward of one accumulated micro-batch: loss gradient scaled by grad_scale first."""
        self._eng._check(self._f["gpt_backward_scaled"](self._g, float(grad_scale)))

    def clip_grad_norm(self, max_norm: float) -> None:
        self._eng._check(self._f["gpt_clip_grad_norm"](self._g, float(max_norm)))

    def train_step_ex(self, accum_steps: int = 1, max_norm: float = 0.0, do_update: bool = True) -> float:
        """One iteration of the reference training loop (src/text_train.cpp:1181-1330)."""
        v = ctypes.c_float()
        self._eng._check(self._f["gpt_train_step_ex"](self._g, int(accum_steps), float(max_norm),
                                                      1 if do_update else 0, ctypes.byref(v)))
        return v.value

    def close(self):
        if getattr(self, "_g", None):
            self._f["gpt_destroy"](self._g)
            self._g = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

"""ctypes binding of the CPU oracle (liboracle.so) and of oracle/_ref.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.  The
product (libnmoe_hip.so and its binding) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_MATH_PATH = os.path.join(HERE, "_ref", "libnmoe_math_ref.so")
REF_STEP_PATH = os.path.join(HERE, "_ref", "libnmoe_cpu_step_ref.so")

HIDDEN, INTER, EXPERTS, GROUP, MAX_K = 2048, 512, 256, 64, 8
EXPERT_SIZE = {4: 1769472, 2: 983040}

_P = C.c_void_p
_I = C.c_int
_SZ = C.c_size_t
_F = C.c_float
_U64 = C.c_uint64
_U32 = C.c_uint32

_ORACLE_SIGS = {
    "orc_bf16_to_f32": (_F, [C.c_uint16]),
    "orc_f32_to_bf16": (C.c_uint16, [_F]),
    "orc_bf16_to_f32_array": (None, [_P, _P, _SZ]),
    "orc_f32_to_bf16_bits": (None, [_P, _P, _SZ]),
    "orc_sigmoid": (_F, [_F]),
    "orc_silu": (_F, [_F]),
    "orc_rms_norm": (None, [_P, _P, _P, _SZ, _F, _I]),
    "orc_softmax": (None, [_P, _SZ]),
    "orc_topk": (_SZ, [_P, _SZ, _SZ, _P, _P]),
    "orc_renormalize": (None, [_P, _SZ]),
    "orc_swiglu": (None, [_P, _P, _P, _SZ]),
    "orc_unpack_row": (None, [_P, _P, _SZ, _I]),
    "orc_dequant_row": (None, [_P, _P, _P, _P, _SZ, _I]),
    "orc_dequant_matvec": (None, [_P, _P, _P, _P, _P, _SZ, _SZ, _I]),
    "orc_route": (_I, [_P, _I, _I, _P, _P, _P]),
    "orc_quantize_rows": (None, [_P, _I, _I, _I, _P, _P, _P]),
    "orc_expf_restated": (_F, [_F]),
    "orc_router_logits_bf16": (None, [_P, _P, _I, _I, _P]),
    "orc_router_logits_q4": (None, [_P, _P, _P, _P, _I, _I, _P]),
    "orc_expert_size": (_SZ, [_I]),
    "orc_expert_offsets": (None, [_I, _P]),
    "orc_expert_gate_up": (None, [_P, _I, _P, _P]),
    "orc_expert_down": (None, [_P, _I, _P, _P]),
    "orc_shared_expert": (None, [_P] * 15),
    "orc_combine": (None, [_P, _P, _P, _I, _P, _P, _P, _I]),
    "orc_moe_step_bf16router": (_I, [_P, _I, _P, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P]),
    "orc_moe_experts": (_I, [_P, _I, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "orc_dispatch": (None, [_P, _I, _I, _I, _I, _P, _P]),
    "orc_moe_layer_rmsnorm": (_I, [_P, _I, _P, _P, _F, _I, _P, _P, _P, _P]),
    "orc_moe_block": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P, _F, _I, _P, _P, _P, _P, _P, _P]),
    "orc_syn_mix64": (_U64, [_U64]),
    "orc_syn_stream": (_U64, [_U64, _U32, _U32, _U32]),
    "orc_syn_rand64": (_U64, [_U64, _U64]),
    "orc_syn_normal": (_F, [_U64, _U64]),
    "orc_syn_expert": (None, [_P, _I, _U64, _U32, _U32, _F]),
    "orc_syn_layer": (None, [_P, _I, _U64, _U32, _F]),
    "orc_syn_bf16_normal": (None, [_P, _SZ, _U64, _U32, _U32, _F]),
    "orc_cpu_step_port": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _P]),
    "orc_cpu_step_bench_port": (C.c_double, [_P, _P, _I, _I, _P, _P, _I, _I, _I, _I, _P]),
    "orc_cpu_tokens_bench_port": (C.c_double, [_P, _I, _P, _P, _P, _I, _I, _I, _P]),
    "orc_cpu_stack_bench_port": (C.c_double, [_P, _P, _I, _I, _I, _P, _I, _I, _F, _I, _P]),
}

_REF_MATH_SIGS = {
    "nmoe_bf16_to_f32": (_F, [C.c_uint16]),
    "nmoe_f32_to_bf16": (C.c_uint16, [_F]),
    "nmoe_cpu_sigmoid": (_F, [_F]),
    "nmoe_cpu_silu": (_F, [_F]),
    "nmoe_cpu_rms_norm": (None, [_P, _P, _P, _SZ, _F, _I]),
    "nmoe_cpu_softmax": (None, [_P, _SZ]),
    "nmoe_cpu_topk": (_SZ, [_P, _SZ, _SZ, _P, _P]),
    "nmoe_cpu_renormalize": (None, [_P, _SZ]),
    "nmoe_cpu_swiglu": (None, [_P, _P, _P, _SZ]),
    "nmoe_cpu_unpack_row": (None, [_P, _P, _SZ, _I]),
    "nmoe_cpu_dequant_row": (None, [_P, _P, _P, _P, _SZ, _I]),
    "nmoe_cpu_dequant_matvec": (None, [_P, _P, _P, _P, _P, _SZ, _SZ, _I]),
    "orc_ref_f32_to_bf16_bits": (None, [_P, _P, _SZ]),
}

_REF_STEP_SIGS = {
    "orc_cpu_step_ref": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _P]),
    "orc_cpu_step_bench_ref": (C.c_double, [_P, _P, _I, _I, _P, _P, _I, _I, _I, _I, _P]),
    "orc_cpu_tokens_bench_ref": (C.c_double, [_P, _I, _P, _P, _P, _I, _I, _I, _P]),
    "orc_cpu_stack_bench_ref": (C.c_double, [_P, _P, _I, _I, _I, _P, _I, _I, _F, _I, _P]),
}

_cache: dict[str, C.CDLL] = {}


def _load(path: str, sigs: dict) -> C.CDLL:
    if path not in _cache:
        h = C.CDLL(path)
        for name, (res, args) in sigs.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _cache[path] = h
    return _cache[path]


def oracle() -> C.CDLL:
    if not os.path.exists(ORACLE_PATH):
        raise FileNotFoundError(f"{ORACLE_PATH} missing: run `make -C oracle`")
    return _load(ORACLE_PATH, _ORACLE_SIGS)


def ref_math() -> C.CDLL | None:
    """The reference's own src/math.m compiled as C (None if not built)."""
    return _load(REF_MATH_PATH, _REF_MATH_SIGS) if os.path.exists(REF_MATH_PATH) else None


def ref_step() -> C.CDLL | None:
    return _load(REF_STEP_PATH, _REF_STEP_SIGS) if os.path.exists(REF_STEP_PATH) else None


def p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---------------------------------------------------------------- helpers

def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """math.m:14-19 round-to-nearest-even (vectorised, same bits)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def syn_layer(bits: int, seed: int, layer: int, sigma: float) -> np.ndarray:
    out = np.empty(EXPERTS * EXPERT_SIZE[bits], dtype=np.uint8)
    oracle().orc_syn_layer(out.ctypes.data, bits, seed, layer, sigma)
    return out


def syn_expert(bits: int, seed: int, layer: int, expert: int, sigma: float) -> np.ndarray:
    out = np.empty(EXPERT_SIZE[bits], dtype=np.uint8)
    oracle().orc_syn_expert(out.ctypes.data, bits, seed, layer, expert, sigma)
    return out


def syn_bf16(n: int, seed: int, layer: int, tag: int, sigma: float) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    oracle().orc_syn_bf16_normal(out.ctypes.data, n, seed, layer, tag, sigma)
    return out


def route(logits: np.ndarray, k: int, want_probs: bool = False):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.zeros(MAX_K, np.uint32)
    w = np.zeros(MAX_K, np.float32)
    probs = np.zeros(lg.size, np.float32) if want_probs else None
    n = oracle().orc_route(lg.ctypes.data, lg.size, k, idx.ctypes.data, w.ctypes.data, p(probs))
    return (idx, w, n, probs) if want_probs else (idx, w, n)


def router_logits_bf16(w_bf16: np.ndarray, x: np.ndarray) -> np.ndarray:
    E = w_bf16.shape[0]
    out = np.zeros(E, np.float32)
    xw = np.ascontiguousarray(x, np.float32)
    oracle().orc_router_logits_bf16(np.ascontiguousarray(w_bf16).ctypes.data, xw.ctypes.data, E, HIDDEN,
                                    out.ctypes.data)
    return out


def moe_experts(pack: np.ndarray, bits: int, x: np.ndarray, k: int, idx: np.ndarray, w: np.ndarray,
                h_mid: np.ndarray, shared_out=None, shared_gate_raw=None, want_act=False):
    ntok = x.shape[0]
    out = np.zeros((ntok, HIDDEN), np.float32)
    act = np.zeros((ntok, MAX_K, INTER), np.float32) if want_act else None
    x = np.ascontiguousarray(x, np.float32)
    rc = oracle().orc_moe_experts(pack.ctypes.data, bits, x.ctypes.data, ntok, k,
                                  np.ascontiguousarray(idx, np.uint32).ctypes.data,
                                  np.ascontiguousarray(w, np.float32).ctypes.data,
                                  np.ascontiguousarray(h_mid, np.float32).ctypes.data,
                                  p(shared_out), p(shared_gate_raw), out.ctypes.data, p(act))
    assert rc == 0
    return (out, act) if want_act else out


def syn_shared_expert(seed: int, sigma: float = 0.02):
    """Synthetic q4 shared-expert tensors: gate/up [512][2048] and down
    [2048][512] are carved out of a generated routed-expert pack (the same
    shapes), score [1][2048] is row 0 of another pack's gate.  Returns
    {name: (w u32, scales u16, biases u16)}."""
    off = [0, 524288, 557056, 589824, 1114112, 1146880, 1179648, 1703936, 1736704, EXPERT_SIZE[4]]
    pk = syn_expert(4, seed, 61, 7, sigma)
    pk2 = syn_expert(4, seed, 61, 8, sigma)
    t = lambda b, i: (b[off[i]:off[i + 1]].view(np.uint32), b[off[i + 1]:off[i + 2]].view(np.uint16),
                      b[off[i + 2]:off[i + 3]].view(np.uint16))
    g2 = t(pk2, 0)
    return {"gate": t(pk, 0), "up": t(pk, 3), "down": t(pk, 6),
            "score": (g2[0][:256].copy(), g2[1][:32].copy(), g2[2][:32].copy())}


def shared_expert(se: dict, x: np.ndarray):
    """orc_shared_expert per token: (shared_out [ntok][2048], shared_gate_raw [ntok])."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    out = np.zeros((x.shape[0], HIDDEN), np.float32)
    g = np.zeros(x.shape[0], np.float32)
    args = [p(np.ascontiguousarray(a)) for n in ("gate", "up", "down", "score") for a in se[n]]
    for t in range(x.shape[0]):
        oracle().orc_shared_expert(*args, x[t].ctypes.data, out[t].ctypes.data, g[t:].ctypes.data)
    return out, g


def quantize_rows(rows_bf16: np.ndarray, bits: int):
    """orc_quantize_rows: (packed u32, scales u16, biases u16)."""
    rows_bf16 = np.ascontiguousarray(rows_bf16, np.uint16)
    rows, cols = rows_bf16.shape
    packed = np.zeros((rows, cols * bits // 32), np.uint32)
    scales = np.zeros((rows, cols // GROUP), np.uint16)
    biases = np.zeros((rows, cols // GROUP), np.uint16)
    oracle().orc_quantize_rows(rows_bf16.ctypes.data, rows, cols, bits, packed.ctypes.data, scales.ctypes.data,
                               biases.ctypes.data)
    return packed, scales, biases


def moe_block(pack: np.ndarray, bits: int, router: dict, h_mid: np.ndarray, k: int, eps: float = 1e-6,
              post_norm=None, add_one: int = 1, shared: dict | None = None, next_norm=None, want_next=False):
    """orc_moe_block for one token.  router: {"w": bf16 [256][2048]} or
    {"q4": (w u32 [256][256], scales, biases)}; shared: syn_shared_expert's
    dict or None.  Returns (out, idx8, w8, x, next_x or None)."""
    h = np.ascontiguousarray(h_mid, np.float32)
    out, x = np.zeros(HIDDEN, np.float32), np.zeros(HIDDEN, np.float32)
    nx = np.zeros(HIDDEN, np.float32) if want_next else None
    idx, w = np.zeros(MAX_K, np.uint32), np.zeros(MAX_K, np.float32)
    keep = []
    if "q4" in router:
        kind, rb = 1, None
        rq = [np.ascontiguousarray(a) for a in router["q4"]]
        keep += rq
        rqp = [a.ctypes.data for a in rq]
    else:
        kind, rb = 0, np.ascontiguousarray(router["w"])
        keep.append(rb)
        rqp = [None, None, None]
    sh = None
    if shared is not None:
        arrs = [np.ascontiguousarray(a) for n in ("gate", "up", "down", "score") for a in shared[n]]
        keep += arrs
        sh = (C.c_void_p * 12)(*[a.ctypes.data for a in arrs])
    rc = oracle().orc_moe_block(pack.ctypes.data, bits, kind, p(rb), rqp[0], rqp[1], rqp[2], sh, p(post_norm),
                                add_one, h.ctypes.data, eps, k, out.ctypes.data, p(next_norm), p(nx),
                                idx.ctypes.data, w.ctypes.data, x.ctypes.data)
    assert rc == 0
    return out, idx, w, x, nx


def dispatch(idx: np.ndarray, ntok: int, k: int, stride: int, num_experts: int = EXPERTS):
    perm = np.zeros(ntok * k, np.uint32)
    offsets = np.zeros(num_experts + 1, np.uint32)
    oracle().orc_dispatch(np.ascontiguousarray(idx, np.uint32).ctypes.data, ntok, k, stride, num_experts,
                          perm.ctypes.data, offsets.ctypes.data)
    return perm, offsets

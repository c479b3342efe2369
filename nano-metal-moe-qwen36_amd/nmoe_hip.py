"""ctypes binding of libnmoe_hip.so (include/nmoe_hip.h) for Python callers.

The library is the product: hand-written gfx950 HIP kernels behind a C ABI.
This module only marshals arguments.  It never computes anything itself and
raises if the shared library is missing: there is no CPU fallback.

Device memory is owned by the library's context (``Context.alloc`` wraps
``nmoe_hip_register_state_buffer``, the counterpart of the reference's
``nmoe_backend_register_state_buffer``, include/nmoe/backend.h:66).  PyTorch
is deliberately not used: its wheel bundles its own HIP runtime, and two HIP
runtimes in one process would not share device pointers.
"""
from __future__ import annotations

import ctypes as C
import itertools
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnmoe_hip.so")
# the phase-timeline build of the same sources (make timeline): the fused
# launches also record their phase boundaries (nmoe_hip_set_timeline)
TIMELINE_LIB_PATH = os.path.join(HERE, "libnmoe_hip_tl.so")
# stamp slots of a fused launch's timeline, in the order the stamps are laid
# out (block b of slot s: stamps[s][b][i] for event TL_EVENTS[i])
TL_EVENTS = ("start", "x_ready", "logit_published", "logits_in", "candidate_0", "candidates", "confirmed",
             "loads_issued", "gate_up_done", "act_published", "act_in", "down_done", "partials_in", "out_written",
             "next_ready", "end")

HIDDEN = 2048
INTER = 512
EXPERTS = 256
GROUP = 64
MAX_K = 8
EXPERT_SIZE = {4: 1769472, 2: 983040}
F32 = 0
BF16 = 1
ROUTER_BF16 = 0
ROUTER_Q4 = 1

OK = 0
EINVAL = -22
ENOMEM = -12
ENODEV = -19
ENOENT = -2
EIO = -5
EHIP = -71
ETIMEDOUT = -110
OPT_FUSED_DECODE = 1
OPT_XCD_LOCAL = 2
OPT_GROUPED_MIN_TOKENS = 3
OPT_SPIN_LIMIT = 4
OPT_SYNC_CHECK = 5
OPT_SKEW_EPOCH = 6
OPT_STACK_LOOP = 7
OPT_GROUPED_ONE_LAUNCH = 8
OPT_SKEW_TILES = 9

# q4 / q2 component offsets (scripts/convert_qwen36.py:38-64)
OFFSETS = {
    4: dict(gate_w=0, gate_s=524288, gate_b=557056, up_w=589824, up_s=1114112, up_b=1146880,
            down_w=1179648, down_s=1703936, down_b=1736704),
    2: dict(gate_w=0, gate_s=262144, gate_b=294912, up_w=327680, up_s=589824, up_b=622592,
            down_w=655360, down_s=917504, down_b=950272),
}


class NmoeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Router(C.Structure):
    _fields_ = [
        ("kind", C.c_int),
        ("num_experts", C.c_int),
        ("w_bf16", C.c_void_p),
        ("w_q4", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
    ]


class QTensor(C.Structure):
    """nmoe_hip_qtensor: a q4 tensor as stored (w u32, scales/biases bf16)."""
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p)]


class SharedExpert(C.Structure):
    """nmoe_hip_shared_expert: gate/up [512][2048], down [2048][512], score [1][2048]."""
    _fields_ = [("gate", QTensor), ("up", QTensor), ("down", QTensor), ("score", QTensor)]


class MoeBlock(C.Structure):
    """nmoe_hip_moe_block: one layer's MoE half (router, shared expert, norms)."""
    _fields_ = [("router", Router), ("has_shared", C.c_int), ("shared", SharedExpert), ("post_norm", C.c_void_p),
                ("next_norm", C.c_void_p), ("add_one", C.c_int), ("eps", C.c_float)]


_lib = None

_P = C.c_void_p
_I = C.c_int
_SIGS = {
    "nmoe_hip_create": (_I, [_I, _I, C.POINTER(_P)]),
    "nmoe_hip_destroy": (None, [_P]),
    "nmoe_hip_last_error": (C.c_char_p, [_P]),
    "nmoe_hip_stream": (_P, [_P]),
    "nmoe_hip_synchronize": (_I, [_P]),
    "nmoe_hip_device_cus": (_I, [_P]),
    "nmoe_hip_check_device_status": (_I, [_P]),
    "nmoe_hip_set_option": (_I, [_P, _I, _I]),
    "nmoe_hip_register_state_buffer": (_I, [_P, C.c_char_p, C.c_size_t, C.POINTER(_P)]),
    "nmoe_hip_register_shared_buffer": (_I, [_P, C.c_char_p, _P, C.c_size_t, C.POINTER(_P)]),
    "nmoe_hip_lookup_buffer": (_P, [_P, C.c_char_p]),
    "nmoe_hip_copy_to_device": (_I, [_P, _P, _P, C.c_size_t]),
    "nmoe_hip_copy_to_host": (_I, [_P, _P, _P, C.c_size_t]),
    "nmoe_hip_expert_size": (C.c_size_t, [_I]),
    "nmoe_hip_upload_layer_pack": (_I, [_P, _I, _I, _P, C.c_size_t]),
    "nmoe_hip_load_layer_file": (_I, [_P, _I, _I, C.c_char_p]),
    "nmoe_hip_layer_pack": (_P, [_P, _I, C.POINTER(_I)]),
    "nmoe_hip_synth_layer_pack": (_I, [_P, _I, _I, C.c_uint64, C.c_float]),
    "nmoe_hip_synth_bf16": (_I, [_P, _P, C.c_size_t, C.c_uint64, C.c_uint32, C.c_uint32, C.c_float, _P]),
    "nmoe_moe_router_logits": (_I, [_P, C.POINTER(Router), _P, _I, _I, _P, _P]),
    "nmoe_moe_topk": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _P]),
    "nmoe_moe_route": (_I, [_P, C.POINTER(Router), _P, _I, _I, _I, _P, _P, _P, _P]),
    "nmoe_moe_experts_q4": (_I, [_P, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "nmoe_moe_experts_q2": (_I, [_P, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "nmoe_moe_layer": (_I, [_P, _I, C.POINTER(Router), _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P]),
    "nmoe_moe_layer_static": (_I, [_P, _I, C.POINTER(Router), _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "nmoe_dequant_rows": (_I, [_P, _I, _P, _P, _P, _I, _I, _P, _P]),
    "nmoe_moe_layer_rmsnorm": (_I, [_P, _I, C.POINTER(Router), _P, C.c_float, _I, _P, _P, _P, _P, _P]),
    "nmoe_moe_stack": (_I, [_P, _I, C.POINTER(_I), C.POINTER(Router), _I, C.c_float, _P, _P, _P, _P]),
    "nmoe_moe_dispatch": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "nmoe_moe_shared_expert": (_I, [_P, C.POINTER(SharedExpert), _P, _I, _I, _P, _P, _P]),
    "nmoe_hip_validate_layout": (_I, [C.c_char_p, C.POINTER(_I), C.POINTER(_I), C.c_char_p, C.c_size_t]),
    "nmoe_hip_load_expert_dir": (_I, [_P, C.c_char_p, _I, C.POINTER(_I), C.POINTER(_I)]),
    "nmoe_moe_block": (_I, [_P, _I, C.POINTER(MoeBlock), _P, _I, _P, _P, _P, _P, _P, _P]),
    "nmoe_hip_load_model_weights": (_I, [_P, C.c_char_p, C.c_char_p, _I, C.POINTER(_I)]),
    "nmoe_hip_layer_block": (_I, [_P, _I, C.POINTER(MoeBlock)]),
    "nmoe_hip_read_probe": (_I, [_P, _P, C.c_size_t, _P, _P]),
    "nmoe_hip_read_probe_grid": (_I, [_P, _P, C.c_size_t, _I, _I, _I, _P, _P]),
    "nmoe_hip_set_timeline": (_I, [_P, _P, _I]),
    "nmoe_moe_experts_from_logits": (_I, [_P, _I, _P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
}


def header_symbols() -> list[str]:
    """Names of every entry point declared in include/nmoe_hip.h."""
    import re
    hdr = os.path.join(os.path.dirname(HERE), "include", "nmoe_hip.h")
    with open(hdr) as f:
        text = f.read()
    return sorted(set(re.findall(r"NMOE_HIP_API\s+[\w\s\*]*?\b(nmoe_\w+)\s*\(", text)))


def use_timeline_build():
    """Loads the phase-timeline build instead of the product build (before
    the first call into either)."""
    global LIB_PATH
    if _lib is not None and LIB_PATH != TIMELINE_LIB_PATH:
        raise RuntimeError("the product library is already loaded")
    LIB_PATH = TIMELINE_LIB_PATH


def lib() -> C.CDLL:
    """Loads libnmoe_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: build it (python -c 'import __graft_entry__ as g; g.build()')")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


class DeviceBuffer:
    """A device allocation owned by a Context (freed at context destroy)."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int, label: str):
        self.ctx, self.ptr, self.nbytes, self.label = ctx, ptr, nbytes, label

    def upload(self, arr: np.ndarray, offset: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload exceeds buffer")
        self.ctx._check(lib().nmoe_hip_copy_to_device(self.ctx.h, self.ptr + offset, a.ctypes.data, a.nbytes))
        return self

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download exceeds buffer")
        self.ctx._check(lib().nmoe_hip_copy_to_host(self.ctx.h, out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def __add__(self, off: int) -> int:
        return self.ptr + off


class Context:
    """One HIP device context of libnmoe_hip.so."""

    _labels = itertools.count()

    def __init__(self, device: int = 0, max_tokens: int = 64):
        h = C.c_void_p()
        rc = lib().nmoe_hip_create(device, max_tokens, C.byref(h))
        if rc != OK:
            raise NmoeError(rc, f"nmoe_hip_create(device={device}, max_tokens={max_tokens}) failed")
        self.h = h
        self.max_tokens = max_tokens

    def close(self):
        if self.h:
            lib().nmoe_hip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc: int) -> int:
        if rc != OK:
            raise NmoeError(rc, self.last_error())
        return rc

    def last_error(self) -> str:
        return lib().nmoe_hip_last_error(self.h).decode()

    @property
    def stream(self) -> int:
        return lib().nmoe_hip_stream(self.h)

    @property
    def cus(self) -> int:
        return lib().nmoe_hip_device_cus(self.h)

    def sync(self):
        self._check(lib().nmoe_hip_synchronize(self.h))

    def set_option(self, option: int, value: int) -> int:
        return lib().nmoe_hip_set_option(self.h, option, int(value))

    def set_fused(self, on: bool):
        self._check(lib().nmoe_hip_set_option(self.h, OPT_FUSED_DECODE, int(bool(on))))

    def set_grouped_min_tokens(self, n: int):
        """Calls with at least n tokens run the grouped (matrix-core) path."""
        self._check(lib().nmoe_hip_set_option(self.h, OPT_GROUPED_MIN_TOKENS, int(n)))

    def set_grouped_one_launch(self, on: bool) -> bool:
        """Gate/up and down of the grouped path in one launch (on) or two;
        False when the device does not allow the one-launch form."""
        rc = lib().nmoe_hip_set_option(self.h, OPT_GROUPED_ONE_LAUNCH, int(bool(on)))
        if rc != OK and on:
            return False
        self._check(rc)
        return True

    def dispatch(self, idx, ntok: int, k: int, perm, offsets, stream=None) -> int:
        return lib().nmoe_moe_dispatch(self.h, _ptr(idx), ntok, k, _ptr(perm), _ptr(offsets), stream)

    def set_xcd_local(self, on: bool):
        """Die-local exchange in the fused launch (raises where the device
        does not deal a launch's blocks round-robin over 8 dies)."""
        self._check(lib().nmoe_hip_set_option(self.h, OPT_XCD_LOCAL, int(bool(on))))

    def device_status(self) -> int:
        return lib().nmoe_hip_check_device_status(self.h)

    def alloc(self, nbytes: int, label: str | None = None) -> DeviceBuffer:
        label = label or f"py{next(self._labels)}"
        p = C.c_void_p()
        self._check(lib().nmoe_hip_register_state_buffer(self.h, label.encode(), nbytes, C.byref(p)))
        return DeviceBuffer(self, p.value, nbytes, label)

    def to_device(self, arr: np.ndarray, label: str | None = None) -> DeviceBuffer:
        a = np.ascontiguousarray(arr)
        return self.alloc(max(a.nbytes, 16), label).upload(a)

    # ---- packs
    def upload_layer(self, layer: int, bits: int, pack: np.ndarray):
        a = np.ascontiguousarray(pack)
        self._check(lib().nmoe_hip_upload_layer_pack(self.h, layer, bits, a.ctypes.data, a.nbytes))

    def load_layer_file(self, layer: int, bits: int, path: str):
        self._check(lib().nmoe_hip_load_layer_file(self.h, layer, bits, path.encode()))

    def synth_layer(self, layer: int, bits: int, seed: int, sigma: float):
        self._check(lib().nmoe_hip_synth_layer_pack(self.h, layer, bits, seed, sigma))

    def synth_bf16(self, buf, n: int, seed: int, layer: int, tag: int, sigma: float, offset: int = 0):
        self._check(lib().nmoe_hip_synth_bf16(self.h, _ptr(buf) + offset, n, seed, layer, tag, sigma, None))

    def layer_pack_ptr(self, layer: int) -> int | None:
        b = C.c_int()
        return lib().nmoe_hip_layer_pack(self.h, layer, C.byref(b))

    def download_expert(self, layer: int, expert: int, bits: int) -> np.ndarray:
        base = self.layer_pack_ptr(layer)
        esz = EXPERT_SIZE[bits]
        out = np.empty(esz, dtype=np.uint8)
        self._check(lib().nmoe_hip_copy_to_host(self.h, out.ctypes.data, base + expert * esz, esz))
        return out

    # ---- routing / experts
    @staticmethod
    def router_bf16(w, num_experts: int = EXPERTS) -> Router:
        return Router(ROUTER_BF16, num_experts, _ptr(w), None, None, None)

    @staticmethod
    def router_q4(w, scales, biases, num_experts: int = EXPERTS) -> Router:
        return Router(ROUTER_Q4, num_experts, None, _ptr(w), _ptr(scales), _ptr(biases))

    def router_logits(self, router: Router, x, x_dtype: int, ntok: int, logits, stream=None) -> int:
        return lib().nmoe_moe_router_logits(self.h, C.byref(router), _ptr(x), x_dtype, ntok, _ptr(logits), stream)

    def topk(self, logits, ntok: int, num_experts: int, k: int, idx, w, probs=None, stream=None) -> int:
        return lib().nmoe_moe_topk(self.h, _ptr(logits), ntok, num_experts, k, _ptr(idx), _ptr(w), _ptr(probs), stream)

    def route(self, router: Router, x, x_dtype: int, ntok: int, k: int, idx, w, logits=None, stream=None) -> int:
        return lib().nmoe_moe_route(self.h, C.byref(router), _ptr(x), x_dtype, ntok, k, _ptr(idx), _ptr(w),
                                    _ptr(logits), stream)

    def experts(self, bits: int, layer: int, x, x_dtype: int, ntok: int, k: int, idx, w, h_mid, out,
                shared_out=None, shared_gate_raw=None, stream=None) -> int:
        fn = lib().nmoe_moe_experts_q4 if bits == 4 else lib().nmoe_moe_experts_q2
        return fn(self.h, layer, _ptr(x), x_dtype, ntok, k, _ptr(idx), _ptr(w), _ptr(h_mid), _ptr(shared_out),
                  _ptr(shared_gate_raw), _ptr(out), stream)

    def moe_layer(self, layer: int, router: Router, x, x_dtype: int, ntok: int, k: int, h_mid, out, idx=None,
                  w=None, logits=None, shared_out=None, shared_gate_raw=None, stream=None) -> int:
        return lib().nmoe_moe_layer(self.h, layer, C.byref(router), _ptr(x), x_dtype, ntok, k, _ptr(h_mid),
                                    _ptr(shared_out), _ptr(shared_gate_raw), _ptr(out), _ptr(idx), _ptr(w),
                                    _ptr(logits), stream)

    def moe_layer_rmsnorm(self, layer: int, router: Router, h_in, eps: float, k: int, h_out, idx=None, w=None,
                          logits=None, stream=None) -> int:
        return lib().nmoe_moe_layer_rmsnorm(self.h, layer, C.byref(router), _ptr(h_in), eps, k, _ptr(h_out),
                                            _ptr(idx), _ptr(w), _ptr(logits), stream)

    def moe_stack(self, layers, routers, k: int, eps: float, h_seq, idx_seq=None, w_seq=None, stream=None) -> int:
        n = len(layers)
        la = (C.c_int * n)(*layers)
        ra = (Router * n)(*routers)
        return lib().nmoe_moe_stack(self.h, n, la, ra, k, eps, _ptr(h_seq), _ptr(idx_seq), _ptr(w_seq), stream)

    def load_expert_dir(self, path: str, nlayers: int = 0):
        """Validates path/layout.json and makes its layer files resident; returns (bits, layers)."""
        b, n = C.c_int(0), C.c_int(0)
        self._check(lib().nmoe_hip_load_expert_dir(self.h, path.encode(), nlayers, C.byref(b), C.byref(n)))
        return b.value, n.value

    @staticmethod
    def shared_expert_desc(gate, up, down, score) -> SharedExpert:
        """Each argument: (w, scales, biases) device buffers or pointers."""
        q = lambda t: QTensor(_ptr(t[0]), _ptr(t[1]), _ptr(t[2]))
        return SharedExpert(q(gate), q(up), q(down), q(score))

    def shared_expert(self, se: SharedExpert, x, x_dtype: int, ntok: int, shared_out, shared_gate_raw,
                      stream=None) -> int:
        return lib().nmoe_moe_shared_expert(self.h, C.byref(se), _ptr(x), x_dtype, ntok, _ptr(shared_out),
                                            _ptr(shared_gate_raw), stream)

    def moe_block(self, layer: int, blk: MoeBlock, h_mid, k: int, out, next_x=None, idx=None, w=None, logits=None,
                  stream=None) -> int:
        return lib().nmoe_moe_block(self.h, layer, C.byref(blk), _ptr(h_mid), k, _ptr(out), _ptr(next_x), _ptr(idx),
                                    _ptr(w), _ptr(logits), stream)

    def load_model_weights(self, bin_path: str, json_path: str, nlayers: int = 0) -> int:
        """Makes the MoE-path tensors of model_weights.bin resident; returns the layer count."""
        n = C.c_int(0)
        self._check(lib().nmoe_hip_load_model_weights(self.h, bin_path.encode(), json_path.encode(), nlayers,
                                                      C.byref(n)))
        return n.value

    def layer_block(self, layer: int) -> MoeBlock:
        b = MoeBlock()
        self._check(lib().nmoe_hip_layer_block(self.h, layer, C.byref(b)))
        return b

    def read_probe(self, src, nbytes: int, sink, stream=None) -> int:
        return lib().nmoe_hip_read_probe(self.h, _ptr(src), nbytes, _ptr(sink), stream)

    def experts_from_logits(self, layer: int, logits, x, x_dtype: int, ntok: int, k: int, h_mid, out, idx, w,
                            shared_out=None, shared_gate_raw=None, stream=None) -> int:
        return lib().nmoe_moe_experts_from_logits(self.h, layer, _ptr(logits), _ptr(x), x_dtype, ntok, k, _ptr(h_mid),
                                                  _ptr(shared_out), _ptr(shared_gate_raw), _ptr(out), _ptr(idx),
                                                  _ptr(w), stream)

    def set_timeline(self, stamps, slots: int) -> int:
        return lib().nmoe_hip_set_timeline(self.h, _ptr(stamps), slots)

    def read_probe_grid(self, src, nbytes: int, blocks: int, threads: int, loads: int, sink, stream=None) -> int:
        return lib().nmoe_hip_read_probe_grid(self.h, _ptr(src), nbytes, blocks, threads, loads, _ptr(sink), stream)

    def dequant_rows(self, bits: int, packed, scales, biases, rows: int, in_dim: int, out, stream=None) -> int:
        return lib().nmoe_dequant_rows(self.h, bits, _ptr(packed), _ptr(scales), _ptr(biases), rows, in_dim,
                                       _ptr(out), stream)


STATIC_MAX_TOKENS = 16


def moe_layer_static(layer_pack, bits: int, router: Router, x, x_dtype: int, ntok: int, k: int, h_mid, out,
                     idx=None, w=None, shared_out=None, shared_gate_raw=None, stream=None) -> int:
    """nmoe_moe_layer_static: the per-layer call with no context and no
    allocation, on the current device (layer_pack: a resident layer's device
    address)."""
    return lib().nmoe_moe_layer_static(_ptr(layer_pack), bits, C.byref(router), _ptr(x), x_dtype, ntok, k,
                                       _ptr(h_mid), _ptr(shared_out), _ptr(shared_gate_raw), _ptr(out), _ptr(idx),
                                       _ptr(w), stream)


def validate_layout(path: str):
    """nmoe_hip_validate_layout: (status, bits, num_layers, message)."""
    b, n = C.c_int(0), C.c_int(0)
    err = C.create_string_buffer(256)
    rc = lib().nmoe_hip_validate_layout(path.encode(), C.byref(b), C.byref(n), err, 256)
    return rc, b.value, n.value, err.value.decode()

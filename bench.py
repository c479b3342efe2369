"""Benchmark: routed-MoE tokens/s and achieved HBM GB/s (q4, top-8, batch 1).

Workload (the headline metric's configuration, on the GPU): one decode
token through one routed-expert layer of Qwen3.6-35B-A3B -- bf16 router
[256][2048], softmax/top-8/renormalise, eight q4 group-64 experts
(2048 -> 512 gate/up, SwiGLU, 512 -> 2048 down), weighted combine into the
fp32 residual.  Steps rotate over 40 synthetic layers resident in HBM
(40 x 453 MB = 18.1 GB, far above the 256 MB last-level cache) and over 320
routers (320 MB), so experts and router rows stream from HBM.  The timed
steps come after the warm-up's, never on the layers it just read.

The same JSON line carries sub-objects measured in the same run: "c2" (the
q2 single-layer step at top-8 and top-6), "c3" (128 decode tokens through
the 40-layer stack, one persistent launch per token), "c4" (64-token batched
decode), "c5" and "c5_q2" (the 2048-token prefill on the grouped
matrix-core path, q4 and q2, with its MFMA utilisation), "block" (the
model's per-layer MoE half, nmoe_moe_block) and "stream" (the streaming
floor of the step's expert bytes, nmoe_hip_read_probe).  Each carries a
cpu_baseline of its own (the per-token configs extrapolated from a token
subset, labelled so).

A step is one call of the per-layer MoE entry point (nmoe_moe_layer), which
for one token is a single persistent launch (nmoe_fused_decode_kernel).
Timed region: `--steps` back-to-back steps on the library's stream,
bracketed by HIP events recorded on that stream and stream synchronisation.
One step is one launch of the dominant kernel, so its average launch
duration for the roofline object is the timed region / steps (this includes
the dispatch gap between back-to-back launches; rocprofv3's kernel-only
average is in profiles/).  `traffic` (HBM bytes per launch) comes from the
rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarised in
profiles/fused_decode_q4_k8.md (copy-calibrated), for the q4 top-8 workload.

Algorithmic bytes per step (q4, K=8): 8 experts x 1,769,472 B + bf16 router
1,048,576 B + activations 20,544 B (x bf16 4 KB, h_mid fp32 8 KB, out fp32
8 KB, idx/w 64 B) = 15,224,896 B.

cpu_baseline: the reference's CPU routines (src/math.m compiled from the
reference sources into oracle/_ref, single-threaded, -O3) on a bounded
sample of the same workload; the repository's C restatement ("port") when
oracle/_ref was not built.

    python bench.py [--gpus 1] [--steps 400] [--warmup 40] [--no-extra] [--workload c1|c3|c4|c5]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "nano-metal-moe-qwen36_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
EXPERT_BYTES = {4: 1769472, 2: 983040}
ROUTER_BYTES = 256 * 2048 * 2
ROUTER_Q4_BYTES = 256 * 256 * 4 + 2 * 256 * 32 * 2  # the model's q4 router: codes + scales + biases
ACT_BYTES = 4096 + 8192 + 8192 + 64


def step_bytes(bits: int, k: int, router: str = "bf16") -> int:
    return k * EXPERT_BYTES[bits] + (ROUTER_BYTES if router == "bf16" else ROUTER_Q4_BYTES) + ACT_BYTES


class HipEvents:
    """hipEvent* through ctypes on the HIP runtime libnmoe_hip.so links."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so.7")
        for n in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                  "hipEventDestroy"):
            getattr(self.rt, n).restype = C.c_int
        self.rt.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.rt.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.rt.hipEventSynchronize.argtypes = [C.c_void_p]
        self.rt.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.rt.hipEventDestroy.argtypes = [C.c_void_p]

    def create(self, n: int) -> list:
        evs = []
        for _ in range(n):
            e = C.c_void_p()
            assert self.rt.hipEventCreate(C.byref(e)) == 0
            evs.append(e)
        return evs

    def record(self, ev, stream):
        assert self.rt.hipEventRecord(ev, stream) == 0

    def ms(self, a, b) -> float:
        assert self.rt.hipEventSynchronize(b) == 0
        out = C.c_float()
        assert self.rt.hipEventElapsedTime(C.byref(out), a, b) == 0
        return float(out.value)

    def copy_d2d(self, dst, src, nbytes, stream):
        """hipMemcpyAsync device-to-device (a blit kernel: the known-size
        copy that HBM byte counters are calibrated against)."""
        f = self.rt.hipMemcpyAsync
        f.restype = C.c_int
        f.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        assert f(dst, src, nbytes, 3, stream) == 0  # hipMemcpyDeviceToDevice

    def destroy(self, evs):
        for e in evs:
            self.rt.hipEventDestroy(e)


class HipGraph:
    """Back-to-back launches captured into one HIP graph (hipStreamBeginCapture
    .. hipGraphInstantiate, through ctypes on the same HIP runtime), so that
    a launch period can be measured without the host's per-launch cost."""

    def __init__(self, rt, stream, issue):
        P = C.c_void_p
        for n, a in (("hipStreamBeginCapture", [P, C.c_int]), ("hipStreamEndCapture", [P, C.POINTER(P)]),
                     ("hipGraphInstantiate", [C.POINTER(P), P, P, C.c_char_p, C.c_size_t]),
                     ("hipGraphLaunch", [P, P]), ("hipGraphExecDestroy", [P]), ("hipGraphDestroy", [P])):
            getattr(rt, n).restype, getattr(rt, n).argtypes = C.c_int, a
        self.rt, self.stream = rt, stream
        self.graph, self.exe = C.c_void_p(), C.c_void_p()
        assert rt.hipStreamBeginCapture(stream, 1) == 0  # thread-local capture mode
        rcs = issue()
        assert rt.hipStreamEndCapture(stream, C.byref(self.graph)) == 0
        assert not any(rcs), rcs
        assert rt.hipGraphInstantiate(C.byref(self.exe), self.graph, None, None, 0) == 0

    def launch(self):
        assert self.rt.hipGraphLaunch(self.exe, self.stream) == 0

    def destroy(self):
        self.rt.hipGraphExecDestroy(self.exe)
        self.rt.hipGraphDestroy(self.graph)


def check_timed(ctx, rcs):
    """After a timed region: every call's status (a call its host-side checks
    rejected launched nothing, so it must not count as a step) and the
    device status word (a bounded wait that gave up)."""
    bad = [(i, rc) for i, rc in enumerate(rcs) if rc != 0]
    if bad:
        raise SystemExit(f"{len(bad)} timed calls failed, first: call {bad[0][0]} returned {bad[0][1]}: "
                         f"{ctx.last_error()}")
    if ctx.device_status() != 0:
        raise SystemExit(f"device status error: {ctx.last_error()}")


KERNEL_SOURCES = ("csrc/fused.hip", "csrc/nmoe_device.h", "csrc/nmoe_exact.h")


def kernel_source_digest() -> str:
    """sha256 over the fused kernel's sources, as the profile summaries record
    it: a summary measured on other sources does not describe this build."""
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(PKG, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def profiled_traffic(bits: int, k: int):
    """HBM bytes per launch from the committed rocprofv3 counter summary of
    this workload: (bytes, True) when the summary was measured on the
    current kernel sources, (None, False) when it was not, (None, None)
    without a summary."""
    path = os.path.join(ROOT, "profiles", f"fused_decode_q{bits}_k{k}.md")
    vals = {}
    try:
        with open(path) as f:
            for line in f:
                for key in ("traffic_bytes_per_launch", "kernel_source_sha256"):
                    if line.startswith(key + " = "):
                        vals[key] = line.split("=", 1)[1].strip()
    except OSError:
        return None, None
    if "traffic_bytes_per_launch" not in vals:
        return None, None
    if vals.get("kernel_source_sha256") != kernel_source_digest():
        return None, False
    return int(vals["traffic_bytes_per_launch"]), True


def cpu_baseline(bits: int, k: int, seed: int, nsteps: int, nlayers: int = 4) -> dict:
    """Times the reference's CPU decode step on `nsteps` steps over `nlayers`
    synthetic layers (only the experts the steps route to are generated)."""
    from oracle import binding as B

    ref = B.ref_step()
    kind = "reference" if ref is not None else "port"
    fn = ref.orc_cpu_step_bench_ref if ref is not None else B.oracle().orc_cpu_step_bench_port
    esz = EXPERT_BYTES[bits]
    sigma = 0.02 if bits == 4 else 0.05
    packs, routers, xs, hs = [], [], [], []
    for layer in range(nlayers):
        W = B.syn_bf16(256 * 2048, seed, layer, 16, 0.02)
        x = B.bf16_to_f32(B.syn_bf16(2048, seed, layer, 17, 1.0))
        h = B.bf16_to_f32(B.syn_bf16(2048, seed, layer, 18, 1.0))
        idx, _, n = B.route(B.router_logits_bf16(W.reshape(256, 2048), x), k)
        pack = np.zeros(256 * esz, np.uint8)
        for e in idx[:n]:
            pack[int(e) * esz:(int(e) + 1) * esz] = B.syn_expert(bits, seed, layer, int(e), sigma)
        packs.append(pack), routers.append(W), xs.append(x), hs.append(h)
    X = np.ascontiguousarray(np.stack(xs))
    H = np.ascontiguousarray(np.stack(hs))
    pp = (C.c_void_p * nlayers)(*[p.ctypes.data for p in packs])
    rp = (C.c_void_p * nlayers)(*[r.ctypes.data for r in routers])
    out = np.zeros(2048, np.float32)
    repeats = 3
    per_rep = max(nlayers, nsteps // repeats)
    t0 = time.time()
    sec = fn(pp, rp, nlayers, bits, X.ctypes.data, H.ctypes.data, nlayers, k, per_rep, repeats, out.ctypes.data)
    wall = time.time() - t0
    tps = 1.0 / sec
    return {
        "value": round(tps, 3),
        "unit": "tokens/s",
        "cores": 1,
        "kind": kind,
        "sample": (f"{repeats}x{per_rep} single-layer q{bits} top-{k} decode steps over {nlayers} synthetic layers "
                   f"(median repeat), {wall:.1f} s of CPU work on 1 of {os.cpu_count()} host threads; "
                   f"{sec * 1e3:.2f} ms/step, {step_bytes(bits, k) / sec / 1e9:.3f} GB/s algorithmic"),
    }


def _cpu_fn(name: str):
    """The CPU routine `name` from oracle/_ref (the reference's math.m) when
    it was built, else from the C restatement: (fn, kind)."""
    from oracle import binding as B
    ref = B.ref_step()
    if ref is not None:
        return getattr(ref, name + "_ref"), "reference"
    return getattr(B.oracle(), name + "_port"), "port"


def cpu_tokens_baseline(bits: int, k: int, seed: int, layer: int, lg: np.ndarray, x: np.ndarray, h: np.ndarray,
                        ntok_step: int, sample: int = 64, repeats: int = 3) -> dict:
    """The batched-decode / prefill configs on the CPU: the reference runs a
    prompt one token at a time (runtime.m:3814-3818), so its per-token time
    on a fixed subset of the step's tokens (given logits, the same synthetic
    layer) extrapolates to the whole step."""
    from oracle import binding as B
    fn, kind = _cpu_fn("orc_cpu_tokens_bench")
    n = min(sample, lg.shape[0])
    lg = np.ascontiguousarray(lg[:n], np.float32)
    x = np.ascontiguousarray(x[:n], np.float32)
    h = np.ascontiguousarray(h[:n], np.float32)
    esz = EXPERT_BYTES[bits]
    pack = np.zeros(256 * esz, np.uint8)
    sel = set()
    for t in range(n):
        idx, _, m = B.route(lg[t], k)
        sel.update(int(e) for e in idx[:m])
    for e in sel:  # only the experts the sample routes to
        pack[e * esz:(e + 1) * esz] = B.syn_expert(bits, seed, layer, e, 0.02 if bits == 4 else 0.05)
    out = np.zeros(2048, np.float32)
    t0 = time.time()
    sec = fn(pack.ctypes.data, bits, lg.ctypes.data, x.ctypes.data, h.ctypes.data, n, k, repeats, out.ctypes.data)
    wall = time.time() - t0
    return {"value": round(1.0 / sec, 3), "unit": "tokens/s", "cores": 1, "kind": kind,
            "sample": (f"{n} of the step's {ntok_step} tokens (layer {layer}, {len(sel)} experts), {repeats} passes, "
                       f"median; one token at a time as the reference's prompt loop; {wall:.1f} s of CPU work on 1 "
                       f"of {os.cpu_count()} host threads; {sec * 1e3:.2f} ms/token, so the {ntok_step}-token step "
                       f"extrapolates to {ntok_step * sec * 1e3:.0f} ms"),
            "extrapolated": True}


def cpu_stack_baseline(bits: int, k: int, seed: int, nl: int, h0: np.ndarray, npacks: int = 2, ntok: int = 1,
                       repeats: int = 3) -> dict:
    """The 40-layer stack on the CPU: x = RMSNorm(h), h += MoE_l(x) for each
    layer, the layers taking `npacks` distinct synthetic layer packs and
    routers in turn (the CPU time per layer does not depend on which)."""
    from oracle import binding as B
    fn, kind = _cpu_fn("orc_cpu_stack_bench")
    sigma = 0.02 if bits == 4 else 0.05
    esz = EXPERT_BYTES[bits]
    packs = []
    for l in range(npacks):
        p = np.empty(256 * esz, np.uint8)
        for e in range(256):
            p[e * esz:(e + 1) * esz] = B.syn_expert(bits, seed, l, e, sigma)
        packs.append(p)
    routers = [B.syn_bf16(256 * 2048, seed, r, 16, 0.02) for r in range(npacks)]
    pp = (C.c_void_p * npacks)(*[p.ctypes.data for p in packs])
    rp = (C.c_void_p * npacks)(*[r.ctypes.data for r in routers])
    h0 = np.ascontiguousarray(h0[:ntok], np.float32)
    out = np.zeros(2048, np.float32)
    t0 = time.time()
    sec = fn(pp, rp, npacks, nl, bits, h0.ctypes.data, ntok, k, 1e-6, repeats, out.ctypes.data)
    wall = time.time() - t0
    return {"value": round(1.0 / sec, 3), "unit": "tokens/s", "cores": 1, "kind": kind,
            "sample": (f"{repeats}x{ntok} tokens through {nl} layers ({npacks} distinct synthetic q{bits} layers in "
                       f"turn), median pass; {wall:.1f} s of CPU work on 1 of {os.cpu_count()} host threads; "
                       f"{sec * 1e3:.1f} ms/token")}


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 (no sparsity)
# Routers rotate over this many copies (320 MB of bf16 routers, above the
# 256 MB memory-side cache), so a step's router row comes from HBM as it does
# in real decode, where the other weights of a token evict the routers.
ROUTER_POOL = 320


def synth_routers(ctx, buf, NR: int, args) -> list:
    """NR synthetic routers in `buf` (NR * ROUTER_BYTES): dense bf16
    N(0, 0.02) [256][2048], or the model's q4 form (codes uniform 0..15,
    scale bf16(N(0, 0.002)), bias bf16(-8 scale), from seeded generators)
    packed into the same slot."""
    rts = []
    for r in range(NR):
        base = buf.ptr + r * ROUTER_BYTES
        if args.router == "bf16":
            ctx.synth_bf16(buf, 256 * 2048, args.seed, r, 16, 0.02, offset=r * ROUTER_BYTES)
            rts.append(ctx.router_bf16(base))
        else:
            rng = np.random.default_rng(args.seed * 1000 + r)
            wq = rng.integers(0, 2**32, size=256 * 256, dtype=np.uint64).astype(np.uint32)
            sc = (rng.standard_normal(256 * 32) * 0.002).astype(np.float32)
            s16 = ((sc.view(np.uint32).astype(np.uint64) + 0x7FFF + ((sc.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
            bi = (-8.0 * (s16.astype(np.uint32) << 16).view(np.float32)).astype(np.float32)
            b16 = ((bi.view(np.uint32).astype(np.uint64) + 0x7FFF + ((bi.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
            buf.upload(wq, offset=r * ROUTER_BYTES)
            buf.upload(s16, offset=r * ROUTER_BYTES + wq.nbytes)
            buf.upload(b16, offset=r * ROUTER_BYTES + wq.nbytes + s16.nbytes)
            rts.append(ctx.router_q4(base, base + wq.nbytes, base + wq.nbytes + s16.nbytes))
    return rts


class Pool:
    """The resident data every workload draws from: NL synthetic layers
    (40 q4 layers = 18.1 GB, far above the memory-side cache), ROUTER_POOL
    routers, and one bf16 x and fp32 residual per router slot."""

    def __init__(self, nh, args, max_tokens: int):
        self.nh, self.args = nh, args
        self.NL, self.NR = args.layers, max(ROUTER_POOL, args.layers)
        bits = args.bits
        self.ctx = ctx = nh.Context(0, max_tokens=max_tokens)
        print(f"[bench] device 0: {ctx.cus} CUs; {self.NL} q{bits} layers, {self.NR} {args.router} routers",
              file=sys.stderr, flush=True)
        for layer in range(self.NL):
            ctx.synth_layer(layer, bits, args.seed, 0.02 if bits == 4 else 0.05)
        self.routers = ctx.alloc(self.NR * ROUTER_BYTES, "bench.routers")
        self.rts = synth_routers(ctx, self.routers, self.NR, args)
        self.X = ctx.alloc(self.NR * 4096, "bench.x")
        Hb = ctx.alloc(self.NR * 4096, "bench.hb")
        ctx.synth_bf16(self.X, self.NR * 2048, args.seed, 0, 17, 1.0)
        ctx.synth_bf16(Hb, self.NR * 2048, args.seed, 0, 18, 1.0)
        hb = Hb.download(np.uint16, (self.NR, 2048))
        self.H = ctx.to_device((hb.astype(np.uint32) << 16).view(np.float32), "bench.h")
        self.h0 = (hb.astype(np.uint32) << 16).view(np.float32)
        ctx.sync()


def run_c1(pool, args) -> dict:
    """The headline: one decode token through one q4 top-8 layer per step.
    Step i uses layer i % 40 and router / x / residual slot i % 320; the
    timed steps are W .. W+K-1, after the K warm-up steps 0 .. W-1, so no
    timed step re-reads a layer or router the warm-up just brought in."""
    nh, ctx, bits, k = pool.nh, pool.ctx, args.bits, args.k
    stream = ctx.stream
    NL, NR = pool.NL, pool.NR
    OUT, IDX, WT = ctx.alloc(NL * 8192), ctx.alloc(NL * 32), ctx.alloc(NL * 32)

    def step(i):
        layer, r = i % NL, i % NR
        return ctx.moe_layer(layer, pool.rts[r], pool.X.ptr + r * 4096, nh.BF16, 1, k, pool.H.ptr + r * 8192,
                             OUT.ptr + layer * 8192, IDX.ptr + layer * 32, WT.ptr + layer * 32, stream=stream)

    for i in range(args.warmup):
        ctx._check(step(i))
    ctx.sync()
    ev = HipEvents()
    e0, e1 = ev.create(2)
    ev.record(e0, stream)
    rcs = [step(args.warmup + i) for i in range(args.steps)]
    ev.record(e1, stream)
    ms = ev.ms(e0, e1) / args.steps
    ctx.sync()
    check_timed(ctx, rcs)
    ev.destroy([e0, e1])
    B = step_bytes(bits, k, args.router)
    achieved = B / (ms * 1e-3) / 1e9
    traffic, current = profiled_traffic(bits, k) if args.router == "bf16" else (None, None)
    return {
        "metric": "routed-MoE tokens/s + achieved HBM GB/s (q4, top-8, batch 1, 1 GPU)",
        "value": round(1e3 / ms, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "hbm_gbps": round(achieved, 1),
        "config": {
            "workload": f"c1: single-layer q{bits} top-{k} batch-1 routed-MoE decode step ({args.router} router, "
                        f"hidden 2048, 256 experts, FFN 512), rotating over {NL} HBM-resident layers and {NR} routers",
            "bits": bits, "k": k, "batch": 1, "layers_rotated": NL, "routers_rotated": NR, "bytes_per_step": B,
            "router": args.router, "entry_point": "nmoe_moe_layer",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_profile_current": current,
            "kernel": f"nmoe_fused_decode_kernel<{bits}, 1, 1> (one launch per step)",
            "kernel_ms": round(ms, 5),
        },
    }


def single_step_summary(r: dict, args, cpu_steps: int) -> dict:
    """A single-layer decode line (run_c1's) as a sub-object, with its own
    CPU baseline."""
    out = {key: r[key] for key in ("value", "unit", "ms_per_step", "hbm_gbps", "roofline", "config")}
    out["metric"] = f"routed-MoE tokens/s (q{args.bits}, top-{args.k}, batch 1, 1 GPU)"
    if not args.no_cpu:
        print(f"[bench] q{args.bits} top-{args.k} cpu baseline ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(args.bits, args.k, args.seed, cpu_steps)
    return out


def run_c3(pool, args, ntok: int = 128) -> dict:
    """C3: 128 decode tokens, each through the 40 resident layers,
    h_{l+1} = h_l + MoE_l(RMSNorm(h_l)) (nmoe_moe_stack); token t takes its
    routers from block t % 8 of the pool (320 MB between reuses).  Four
    untimed tokens with their own inputs go first."""
    nh, ctx, bits, k, NL = pool.nh, pool.ctx, args.bits, args.k, pool.NL
    stream = ctx.stream
    ctx._check(ctx.set_option(nh.OPT_STACK_LOOP, args.stack_loop))
    sets = pool.NR // NL
    layers = list(range(NL))
    row = (NL + 1) * 2048 * 4
    warm = 4
    HS = ctx.alloc((ntok + warm) * row, "c3.hseq")
    for t in range(ntok + warm):
        HS.upload(pool.h0[t % pool.NR], offset=t * row)
    ctx.sync()

    def step(t):
        rs = [pool.rts[(t % sets) * NL + l] for l in layers]
        return ctx.moe_stack(layers, rs, k, 1e-6, HS.ptr + t * row, stream=stream)

    for t in range(ntok, ntok + warm):
        ctx._check(step(t))
    ctx.sync()
    ev = HipEvents()
    e0, e1 = ev.create(2)
    ev.record(e0, stream)
    rcs = [step(t) for t in range(ntok)]
    ev.record(e1, stream)
    ms = ev.ms(e0, e1) / ntok
    ctx.sync()
    check_timed(ctx, rcs)
    ev.destroy([e0, e1])
    B = NL * step_bytes(bits, k, args.router)
    gbs = B / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu and args.router == "bf16":
        print("[bench] c3 cpu baseline ...", file=sys.stderr, flush=True)
        cpu = cpu_stack_baseline(bits, k, args.seed, NL, pool.h0)
    return {
        "cpu_baseline": cpu,
        "metric": f"routed-MoE stack tokens/s (c3: {NL} layers, q{bits}, top-{k}, batch 1, 1 GPU)",
        "value": round(1e3 / ms, 1), "unit": "tokens/s", "tokens": ntok, "ms_per_token": round(ms, 5),
        "us_per_layer": round(ms * 1e3 / NL, 2), "hbm_gbps": round(gbs, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4)},
        "config": {"workload": "c3", "layers": NL, "bits": bits, "k": k, "bytes_per_token": B, "router": args.router,
                   "routers_rotated": pool.NR, "entry_point": "nmoe_moe_stack",
                   "launches_per_token": -(-NL // 64) if args.stack_loop else NL},
    }


def run_grouped(pool, args, workload: str, NLg: int = 8) -> dict:
    """C4 (64 tokens, Zipf-skewed logits = ln p_e + Gumbel, p_e ~ rank^-1.1)
    or C5 (2048 tokens, uniform U(0,1) logits): a step is the routing from
    the given logits (math.m softmax / top-k / renormalise) + the grouped
    expert path (dispatch, gate/up + SwiGLU and down on the matrix cores,
    slot-order combine), by default one nmoe_moe_experts_from_logits call.  Timed steps rotate
    over layers 0 .. NLg-1; the warm-up runs layers NLg .. 2 NLg - 1 first."""
    nh, ctx, bits, k = pool.nh, pool.ctx, args.bits, args.k
    stream = ctx.stream
    ntok = 64 if workload == "c4" else 2048
    rng = np.random.default_rng(args.seed + (4 if workload == "c4" else 5))
    logits, xs, hs, touched = [], [], [], []
    for layer in range(2 * NLg):
        if workload == "c4":
            order = rng.permutation(256)
            logp = np.empty(256)
            logp[order] = -1.1 * np.log(np.arange(1, 257))
            lg = (logp[None, :] + rng.gumbel(size=(ntok, 256))).astype(np.float32)
        else:
            lg = rng.random((ntok, 256), dtype=np.float32)
        xb = np.ascontiguousarray(
            (rng.standard_normal((ntok, 2048)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
        hf = rng.standard_normal((ntok, 2048)).astype(np.float32)
        if layer == 0:
            host0 = (lg, (xb.astype(np.uint32) << 16).view(np.float32), hf)
        logits.append(ctx.to_device(lg))
        xs.append(ctx.to_device(xb))
        hs.append(ctx.to_device(hf))
        top = np.argsort(-lg, axis=1, kind="stable")[:, :k]
        touched.append(len(np.unique(top)))
    IDX, WT, OUT = ctx.alloc(ntok * 32), ctx.alloc(ntok * 32), ctx.alloc(ntok * 2048 * 4)
    # the library runs gate/up and down in one launch where the device allows
    # it and the experts average at most half a 64-entry pass (one pass lane:
    # ntok * k <= 8192), else in two
    one = args.grouped_launches == 1 and ctx.set_grouped_one_launch(True) and ntok * k <= 8192
    if args.grouped_launches == 2:
        ctx.set_grouped_one_launch(False)
    ctx.sync()

    def step(layer):
        if args.grouped_entry == "from-logits":
            ctx._check(ctx.experts_from_logits(layer, logits[layer], xs[layer], nh.BF16, ntok, k, hs[layer], OUT, IDX,
                                               WT, stream=stream))
        else:
            ctx._check(ctx.topk(logits[layer], ntok, 256, k, IDX, WT, stream=stream))
            ctx._check(ctx.experts(bits, layer, xs[layer], nh.BF16, ntok, k, IDX, WT, hs[layer], OUT, stream=stream))

    steps = 100 if workload == "c4" else 30
    for i in range(2 * NLg):
        step(NLg + i % NLg)
    ctx.sync()
    if args.timeline:
        return grouped_timeline(ctx, step, NLg, workload, one, dump=args.timeline_dump)
    ev = HipEvents()
    e0, e1 = ev.create(2)
    ev.record(e0, stream)
    for i in range(steps):
        step(i % NLg)
    ev.record(e1, stream)
    ms = ev.ms(e0, e1) / steps
    ctx.sync()
    if ctx.device_status() != 0:
        raise SystemExit(f"device status error: {ctx.last_error()}")
    ev.destroy([e0, e1])
    ctx.set_grouped_one_launch(True)
    cpu = None
    if not args.no_cpu:
        print(f"[bench] {workload} q{bits} cpu baseline ...", file=sys.stderr, flush=True)
        cpu = cpu_tokens_baseline(bits, k, args.seed, 0, *host0, ntok_step=ntok)
    esz = EXPERT_BYTES[bits]
    U = float(np.mean([touched[i % NLg] for i in range(steps)]))
    act_bytes = ntok * (4096 + 8192 + 8192 + 64) + ntok * 256 * 4  # x, h, out, idx/w, logits
    B = U * esz + act_bytes
    flops = 2.0 * ntok * k * 3 * 2048 * 512
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = B / (ms * 1e-3) / 1e9
    return {
        "cpu_baseline": cpu,
        "metric": f"routed-MoE tokens/s ({workload}: {ntok} tokens, q{bits}, top-{k}, 1 GPU)",
        "value": round(ntok / (ms * 1e-3), 1), "unit": "tokens/s", "steps": steps, "ms_per_step": round(ms, 5),
        "dtype": "bf16 x (exact integer codes) on the matrix cores, fp32 accumulate",
        "hbm_gbps": round(gbs, 1), "roofline_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "mfma_tflops": round(tflops, 1), "mfma_utilisation": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        "roofline": {"bound": "mfma" if workload == "c5" else "hbm",
                     "achieved": round(tflops, 1) if workload == "c5" else round(gbs, 1),
                     "peak": MFMA_BF16_PEAK_TFLOPS if workload == "c5" else HBM_PEAK_GBS,
                     "unit": "TFLOP/s" if workload == "c5" else "GB/s",
                     "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS if workload == "c5" else gbs / HBM_PEAK_GBS, 4)},
        "config": {"workload": workload, "tokens": ntok, "bits": bits, "k": k, "layers_rotated": NLg,
                   "distinct_experts_per_step": round(U, 1), "bytes_per_step": int(B), "flops_per_step": int(flops),
                   "entry_point": ("nmoe_moe_experts_from_logits (routing in the grouped path's first launch)"
                                   if args.grouped_entry == "from-logits"
                                   else "nmoe_moe_topk + nmoe_moe_experts_q%d (grouped path)" % bits),
                   "gemm_launches": 1 if one else 2},
    }


GTL_SLOTS = 16  # timeline slots of one grouped step: 4 stamps a block, 1,024 blocks a slot


def grouped_timeline(ctx, step, NLg: int, workload: str, one: bool, nsteps: int = 8, dump: str = "") -> dict:
    """Block timeline of the grouped GEMM launches (timeline build): for
    nsteps steps, each block of the gate/up and down launches (or of the one
    launch) records its start, the end of its wait (down tiles of the
    one-launch form) and its end.  Per step, from the first block's start:
    the blocks with work of each kind (count, median duration, median
    wait), when the last gate/up tile ends and the first down tile starts,
    the GEMMs' span, and the mean number of blocks with work running at once
    over that span (two a CU can run: 512).  The preparation launch's blocks
    record theirs too: when its routing, dispatch and x-plane blocks are
    ready and end, from its first block's start, and the gap from its last
    block's end to the GEMM launch's first block."""
    tick_us = 0.01  # s_memrealtime counts at 100 MHz
    words = GTL_SLOTS * 256 * 16
    stamps = ctx.alloc(words * 8)
    per, raw = [], []
    for i in range(nsteps):
        stamps.upload(np.zeros(words, np.uint64))
        # an unstamped step first, so that the stamped one follows a step on the GPU as in the timed loop
        # (the first launch after the copy and the synchronisation starts its blocks on the dies over several us)
        step((i + NLg - 1) % NLg)
        ctx._check(ctx.set_timeline(stamps, GTL_SLOTS))
        step(i % NLg)
        ctx.sync()
        ctx._check(ctx.set_timeline(None, 0))
        r = stamps.download(np.uint64, (words // 4, 4))
        r = r[r[:, 0] > 0].astype(np.int64)
        raw.append(r)
        info = r[:, 3]
        work, kind = info >> 32, (info >> 28) & 15
        gemm = (kind == 1) | (kind == 2)
        t0 = r[gemm, 0].min()  # the GEMM launch's first block (preparation blocks start before it)
        st, rd, en = (r[:, 0] - t0) * tick_us, (r[:, 1] - t0) * tick_us, (r[:, 2] - t0) * tick_us
        gu, dn = (work > 0) & (kind == 1), (work > 0) & (kind == 2)  # gate/up and down tiles with work
        span = float(en[gu | dn].max())
        # the preparation launch, from its first block's start: routing blocks (their first token
        # routed and counted), the dispatch block (its slice routed; its end), the x-plane blocks
        pr, pd, px = kind == 3, kind == 4, kind == 5
        p0 = st[pr | pd | px].min()
        prep = {
            "prep_route_ready_median_us": float(np.median(rd[pr] - p0)) if pr.any() else None,
            "prep_route_end_max_us": float((en[pr] - p0).max()) if pr.any() else None,
            "prep_dispatch_ready_us": float((rd[pd] - p0).max()), "prep_dispatch_end_us": float((en[pd] - p0).max()),
            "prep_x_end_max_us": float((en[px] - p0).max()) if px.any() else None,
            "prep_span_us": float((en[pr | pd | px] - p0).max()),
            "prep_end_to_gemm_start_us": float(-en[pr | pd | px].max()),
        }
        grid = np.arange(0.0, span, 0.25)
        busy = ((st[gu | dn][None, :] <= grid[:, None]) & (grid[:, None] < en[gu | dn][None, :])).sum(axis=1)
        per.append({
            "span_us": span, "gateup_blocks": int(gu.sum()), "down_blocks": int(dn.sum()),
            "gateup_median_us": float(np.median(en[gu] - st[gu])), "down_median_us": float(np.median(en[dn] - st[dn])),
            "down_wait_median_us": float(np.median(rd[dn] - st[dn])), "down_wait_max_us": float((rd[dn] - st[dn]).max()),
            "last_gateup_end_us": float(en[gu].max()), "first_down_start_us": float(st[dn].min()),
            "busy_mean": float(busy.mean()), "busy_after_last_gateup_start_mean":
                float(busy[grid >= st[gu].max()].mean()) if (grid >= st[gu].max()).any() else None,
            **prep,
        })
    if dump:  # the raw block records: [start, ready, end, info] ticks per block, one array per step
        np.savez_compressed(dump, *raw)
    med = {key: (round(float(np.median([p[key] for p in per])), 3) if per[0][key] is not None else None) for key in per[0]}
    for key, v in med.items():
        print(f"[timeline] {workload} {key:36s} {v}", file=sys.stderr, flush=True)
    return {"metric": f"block timeline of the {workload} grouped GEMM launches (timeline build)", "workload": workload,
            "gemm_launches": 1 if one else 2, "steps": nsteps, "medians": med}


BLOCK_SLOTS = 160  # per-layer model tensors rotated by the block workload: 160 x 2.1 MB, above the 256 MB MALL


def _block_tensors(rng, ns: int):
    """ns slots of one layer's MoE-half model tensors in their stored form,
    each tensor 256-byte aligned inside its slot: q4 router [256][2048],
    shared gate/up [512][2048], down [2048][512] and gate score [1][2048]
    (codes uniform 0..15, scales bf16(N(0, sigma)), biases bf16(-8 scale)),
    then the post-attention and next-layer norm weights (bf16, N(0, 0.1)).
    Returns (uint8 [ns][slot bytes], {name: [offsets in a slot]})."""
    def bf16(v):
        u = v.astype(np.float32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    shapes = {"router": (256, 2048, 0.002), "gate": (512, 2048, 0.002), "up": (512, 2048, 0.002),
              "down": (2048, 512, 0.004), "score": (1, 2048, 0.002)}
    offs, pos = {}, 0
    al = lambda n: (n + 255) // 256 * 256
    for name, (r, c, _) in shapes.items():
        offs[name] = [pos, pos + al(r * c // 2), pos + al(r * c // 2) + al(r * c // 32)]
        pos = offs[name][2] + al(r * c // 32)
    offs["norm"] = [pos, pos + al(4096)]
    slot = pos + 2 * al(4096)
    buf = np.zeros((ns, slot), np.uint8)
    for name, (r, c, sigma) in shapes.items():
        w0, s0, b0 = offs[name]
        buf[:, w0:w0 + r * c // 2] = rng.integers(0, 256, size=(ns, r * c // 2), dtype=np.uint8)
        sc = bf16(rng.standard_normal((ns, r * c // 64)) * sigma)
        bi = bf16(-8.0 * (sc.astype(np.uint32) << 16).view(np.float32))
        buf[:, s0:s0 + r * c // 32] = sc.view(np.uint8).reshape(ns, -1)
        buf[:, b0:b0 + r * c // 32] = bi.view(np.uint8).reshape(ns, -1)
    for i in range(2):
        buf[:, offs["norm"][i]:offs["norm"][i] + 4096] = bf16(rng.standard_normal((ns, 2048)) * 0.1).view(np.uint8)
    return buf, offs


def run_block(pool, args) -> dict:
    """The model's per-layer MoE half as the drop-in runs it (nmoe_moe_block):
    post-attention RMSNorm (1 + w), the q4 router, the shared expert (q4
    gate/up/down and gate score), the routed experts, the combine and the
    next layer's input norm, one launch per layer.  Step i runs the experts
    of layer i % 40 with model-tensor slot i % 160 (router, shared expert,
    norms: 160 x 2.1 MB, more than the memory-side cache holds) on residual
    slot i % 320, after the warm-up's steps."""
    nh, ctx, bits, k, NL = pool.nh, pool.ctx, args.bits, args.k, pool.NL
    stream = ctx.stream
    NS = max(BLOCK_SLOTS, NL)
    buf, offs = _block_tensors(np.random.default_rng(args.seed * 7919 + 11), NS)
    dev = ctx.to_device(buf, "bench.block")
    slot = buf.shape[1]
    blks = []
    for i in range(NS):
        P = lambda name: [dev.ptr + i * slot + o for o in offs[name]]
        se = ctx.shared_expert_desc(P("gate"), P("up"), P("down"), P("score"))
        n0, n1 = P("norm")
        blks.append(nh.MoeBlock(ctx.router_q4(*P("router")), 1, se, n0, n1, 1, 1e-6))
    out, nx, di, dw = ctx.alloc(8192), ctx.alloc(8192), ctx.alloc(32), ctx.alloc(32)
    ctx.sync()

    def step(i):
        ctx._check(ctx.moe_block(i % NL, blks[i % NS], pool.H.ptr + (i % pool.NR) * 8192, k, out, nx, di, dw,
                                 stream=stream))

    for i in range(args.warmup):
        step(i)
    ctx.sync()
    if ctx.device_status() != 0:
        raise SystemExit(f"device status error: {ctx.last_error()}")
    ev = HipEvents()
    e0, e1 = ev.create(2)
    ev.record(e0, stream)
    for i in range(args.steps):
        step(args.warmup + i)
    ev.record(e1, stream)
    ms = ev.ms(e0, e1) / args.steps
    ctx.sync()
    if ctx.device_status() != 0:
        raise SystemExit(f"device status error: {ctx.last_error()}")
    ev.destroy([e0, e1])
    shared_bytes = 2 * (512 * 1024 + 2 * 512 * 32 * 2) + (2048 * 256 + 2 * 2048 * 8 * 2) + (1024 + 2 * 32 * 2)
    B = k * EXPERT_BYTES[bits] + ROUTER_Q4_BYTES + shared_bytes + 2 * 4096 + 3 * 8192 + 64
    gbs = B / (ms * 1e-3) / 1e9
    return {"metric": f"routed-MoE block tokens/s (the model's per-layer MoE half: q4 router, shared expert, "
                      f"norms; q{bits}, top-{k}, batch 1, 1 GPU)",
            "value": round(1e3 / ms, 1), "unit": "tokens/s", "us_per_layer": round(ms * 1e3, 3),
            "hbm_gbps": round(gbs, 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "config": {"workload": "block", "layers_rotated": NL, "tensor_slots_rotated": NS, "bits": bits, "k": k,
                       "bytes_per_step": B, "entry_point": "nmoe_moe_block"}}


def run_stream(pool, args) -> dict:
    """The streaming ceiling of the c1 step: nmoe_hip_read_probe over the
    bytes of 8 q4 experts (14,155,776 B), all loads in flight at once, one
    launch per step, rotating over the 40 layers (no reuse within 18 GB)."""
    ctx, stream = pool.ctx, pool.ctx.stream
    nbytes = 8 * EXPERT_BYTES[args.bits]
    sink = ctx.alloc(2048 * 4, "stream.sink")
    packs = [ctx.layer_pack_ptr(l) for l in range(pool.NL)]

    def step(i):
        ctx._check(ctx.read_probe(packs[i % pool.NL] + ((i // pool.NL) % 8) * nbytes, nbytes, sink, stream=stream))

    for i in range(args.warmup):
        step(i)
    ctx.sync()
    ev = HipEvents()
    e0, e1 = ev.create(2)
    ev.record(e0, stream)
    for i in range(args.steps):
        step(args.warmup + i)
    ev.record(e1, stream)
    ms = ev.ms(e0, e1) / args.steps
    ctx.sync()
    ev.destroy([e0, e1])
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"metric": "streaming ceiling of the c1 step's expert bytes (read probe, 1 GPU)", "value": round(gbs, 1),
            "unit": "GB/s", "us_per_launch": round(ms * 1e3, 3), "bytes": nbytes, "steps": args.steps,
            "frac": round(gbs / HBM_PEAK_GBS, 4), "config": {"workload": "stream", "entry_point": "nmoe_hip_read_probe"}}


def run_timeline(pool, args) -> dict:
    """The phase timeline of a fused workload from the timeline build of the
    library (libnmoe_hip_tl.so, bench.py --timeline): `--steps` launches (c1,
    block) or 16 tokens of 40 layers (c3) record the device clock at each
    block's phase boundaries.  Per launch (per layer for c3), times are taken
    from the first block's start; each event's figure is the median over the
    launches of the median over the blocks that record it ("median_us") and
    of the latest block ("latest_us")."""
    nh, ctx, k = pool.nh, pool.ctx, args.k
    stream = ctx.stream
    wl = args.workload
    ev = HipEvents()
    e0, e1 = ev.create(2)
    if wl == "c3":
        ctx._check(ctx.set_option(nh.OPT_STACK_LOOP, 1))
        NL, ntok = pool.NL, 16
        row = (NL + 1) * 2048 * 4
        HS = ctx.alloc((ntok + 2) * row)
        for t in range(ntok + 2):
            HS.upload(pool.h0[t % pool.NR], offset=t * row)
        step = lambda t: ctx.moe_stack(list(range(NL)), [pool.rts[(t % 8) * NL + l] for l in range(NL)], k, 1e-6,
                                       HS.ptr + t * row, stream=stream)
        warm, timed, per = [ntok, ntok + 1], list(range(ntok)), NL
    elif wl == "block":
        NS = max(BLOCK_SLOTS, pool.NL)
        buf, offs = _block_tensors(np.random.default_rng(args.seed * 7919 + 11), NS)
        dev = ctx.to_device(buf)
        slot = buf.shape[1]
        blks = []
        for i in range(NS):
            P = lambda name: [dev.ptr + i * slot + o for o in offs[name]]
            blks.append(nh.MoeBlock(ctx.router_q4(*P("router")), 1,
                                    ctx.shared_expert_desc(P("gate"), P("up"), P("down"), P("score")),
                                    *P("norm"), 1, 1e-6))
        out, nx = ctx.alloc(8192), ctx.alloc(8192)
        step = lambda i: ctx.moe_block(i % pool.NL, blks[i % NS], pool.H.ptr + (i % pool.NR) * 8192, k, out, nx,
                                       stream=stream)
        warm, timed, per = list(range(args.warmup)), [args.warmup + i for i in range(args.steps)], 1
    else:
        OUT = ctx.alloc(pool.NL * 8192)
        step = lambda i: ctx.moe_layer(i % pool.NL, pool.rts[i % pool.NR], pool.X.ptr + (i % pool.NR) * 4096, nh.BF16,
                                       1, k, pool.H.ptr + (i % pool.NR) * 8192, OUT.ptr + (i % pool.NL) * 8192,
                                       stream=stream)
        warm, timed, per = list(range(args.warmup)), [args.warmup + i for i in range(args.steps)], 1
    slots = len(timed) * per
    stamps = ctx.alloc(slots * 256 * 16 * 8)
    stamps.upload(np.zeros(slots * 256 * 16, np.uint64))
    for i in warm:
        ctx._check(step(i))
    ctx.sync()
    ctx._check(ctx.set_timeline(stamps, slots))
    ev.record(e0, stream)
    rcs = [step(i) for i in timed]
    ev.record(e1, stream)
    ms = ev.ms(e0, e1)
    ctx.sync()
    check_timed(ctx, rcs)
    ctx._check(ctx.set_timeline(None, 0))
    ev.destroy([e0, e1])
    st = stamps.download(np.uint64, (slots, 256, 16)).astype(np.int64)
    have = st > 0
    t0 = np.where(have[:, :, 0], st[:, :, 0], np.iinfo(np.int64).max).min(axis=1)  # each slot's first block start
    span = int(st[have].max() - t0.min())
    mhz = span / (ms * 1e3)  # clock ticks per microsecond over the timed region (the region adds the launch gaps)
    tick_us = 0.01  # s_memrealtime counts at 100 MHz on this part
    events = {}
    for i, name in enumerate(nh.TL_EVENTS):
        med, late = [], []
        for sl in range(slots):
            v = st[sl, have[sl, :, i], i]
            if v.size:
                rel = (v - t0[sl]) * tick_us
                med.append(float(np.median(rel)))
                late.append(float(rel.max()))
        if med:
            events[name] = {"median_us": round(float(np.median(med)), 3), "latest_us": round(float(np.median(late)), 3),
                            "blocks": int(have[:, :, i].sum() // slots)}
    period = None
    if per > 1:  # c3: the layer period, start to start within a launch
        starts = t0.reshape(len(timed), per)
        period = round(float(np.median(np.diff(starts, axis=1))) * tick_us, 3)
    for name, e in events.items():
        print(f"[timeline] {name:16s} median {e['median_us']:7.3f} us  latest {e['latest_us']:7.3f} us  "
              f"({e['blocks']} blocks)", file=sys.stderr, flush=True)
    return {"metric": f"phase timeline of the {wl} fused launch (timeline build)", "workload": wl,
            "launches": len(timed), "slots": slots, "ms_timed_region": round(ms, 4),
            "us_per_launch": round(ms * 1e3 / len(timed), 3), "layer_period_us": period,
            "stamp_ticks_per_us_over_region": round(mhz, 2), "events": events}


SWEEP_POOL = 9 << 29  # 4.5 GiB of synthetic words the sweep's reads rotate over


def run_probe_sweep(nh, args) -> dict:
    """The part's streaming ceiling against size and launch shape
    (nmoe_hip_read_probe_grid), the counterpart of the reference's
    scripts/matvec_bench.m sweep: each size read back to back from offsets
    rotating over a 4.5 GiB pool (no launch re-reads what the one before it
    read, and each size beyond the 256 MB memory-side cache comes from HBM),
    at 256 .. 2048 blocks and 4 .. 16 loads a thread a round; then the
    period of a near-empty launch (16 bytes) of 256 .. 1024 blocks.  HIP
    events around the launches of each point; the median of three repeats."""
    ctx = nh.Context(0, max_tokens=1)
    stream = ctx.stream
    buf = ctx.alloc(SWEEP_POOL, "sweep.pool")
    ctx.synth_bf16(buf, SWEEP_POOL // 2, args.seed, 0, 21, 1.0)
    sink = ctx.alloc(8192 * 1024 // 64 * 4, "sweep.sink")
    ctx.sync()
    ev = HipEvents()
    e = ev.create(2)

    def point(nbytes, blocks, threads, loads, launches, graph=False):
        span = SWEEP_POOL - nbytes
        stride = (nbytes + 4095) // 4096 * 4096 + 4096
        offs = [(i * stride) % max(span, 1) // 4096 * 4096 for i in range(3 * launches + 2)]
        issue = lambda i: ctx.read_probe_grid(buf.ptr + offs[i], nbytes, blocks, threads, loads, sink, stream=stream)
        for i in range(2):
            ctx._check(issue(i))
        graphs = [HipGraph(ev.rt, stream, lambda r=r: [issue(2 + r * launches + i) for i in range(launches)])
                  for r in range(3)] if graph else None
        reps = []
        for r in range(3):
            ev.record(e[0], stream)
            if graph:
                graphs[r].launch()
                rcs = []
            else:
                rcs = [issue(2 + r * launches + i) for i in range(launches)]
            ev.record(e[1], stream)
            reps.append(ev.ms(e[0], e[1]) / launches)
            check_timed(ctx, rcs)
        for gr in graphs or ():
            gr.destroy()
        ms = sorted(reps)[1]
        gbs = nbytes / (ms * 1e-3) / 1e9
        row = {"bytes": nbytes, "blocks": blocks, "threads": threads, "loads": loads, "launches": launches,
               "launch": "graph" if graph else "eager",
               "us_per_launch": round(ms * 1e3, 3), "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        print(f"[sweep] {json.dumps(row)}", file=sys.stderr, flush=True)
        return row

    rows = []
    step_bytes_q4 = 8 * EXPERT_BYTES[4]
    sizes = [(step_bytes_q4, 200), (64 << 20, 60), (256 << 20, 20), (1 << 30, 8), (4 << 30, 3)]
    for nbytes, launches in sizes:
        for blocks in (256, 512, 1024, 2048):
            for loads in (4, 8, 16):
                rows.append(point(nbytes, blocks, 512, loads, launches))
    for threads in (256, 1024):  # the step's size at other block sizes
        for blocks in (256, 512, 1024):
            rows.append(point(step_bytes_q4, blocks, threads, 8, 200))
    for blocks in (256, 512, 1024):  # the step's size, the launches in one graph (no host cost per launch)
        rows.append(point(step_bytes_q4, blocks, 512, 8, 200, graph=True))
    empty = []
    for graph in (False, True):
        for blocks in (256, 512, 1024):
            for threads in (64, 512, 1024):
                r = point(16, blocks, threads, 1, 400, graph=graph)
                empty.append({k: r[k] for k in ("blocks", "threads", "launch", "us_per_launch")})
    ev.destroy(e)
    ctx.close()
    step_rows = [r for r in rows if r["bytes"] == step_bytes_q4 and r["launch"] == "eager"]
    best_step = min(step_rows, key=lambda r: r["us_per_launch"])
    big = [r for r in rows if r["bytes"] >= 1 << 30]
    best_big = max(big, key=lambda r: r["gbs"])
    return {"metric": "streaming read ceiling against size and launch shape (read probe, 1 GPU)",
            "unit": "GB/s", "value": best_big["gbs"],
            "sustained_best": best_big, "step_bytes_best": best_step, "points": rows, "empty_launch": empty,
            "config": {"workload": "probe-sweep", "pool_bytes": SWEEP_POOL, "entry_point": "nmoe_hip_read_probe_grid"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--bits", type=int, default=4, choices=(4, 2))
    ap.add_argument("--k", type=int, default=8)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-steps", type=int, default=630)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--stack-loop", type=int, default=1, choices=(0, 1),
                    help="c3: the token's layers in one persistent launch (1, default) or one launch per layer (0)")
    ap.add_argument("--no-extra", action="store_true", help="c1 only: no c3 / c4 / c5 / stream / block sub-objects")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (counter calibration) and exit")
    ap.add_argument("--grouped-entry", default="from-logits", choices=("from-logits", "topk+experts"),
                    help="c4 / c5: one call routing from the given logits inside the grouped path (default), or "
                         "nmoe_moe_topk then nmoe_moe_experts")
    ap.add_argument("--grouped-launches", type=int, default=1, choices=(1, 2),
                    help="c4 / c5: gate/up and down of the grouped path in one launch (1, default, where the device's "
                         "die placement allows it) or two")
    ap.add_argument("--timeline", action="store_true",
                    help="c1 / c3 / block: load the phase-timeline build (libnmoe_hip_tl.so) and print the medians of "
                         "each phase boundary instead of the bench line; c4 / c5: the block timeline of the grouped "
                         "GEMM launches")
    ap.add_argument("--timeline-dump", default="", metavar="PATH",
                    help="c4 / c5 with --timeline: also write the raw block records to PATH (.npz)")
    ap.add_argument("--router", default="bf16", choices=("bf16", "q4"),
                    help="c1/c3: the benchmark configs' dense bf16 router (default) or the model's q4 router")
    ap.add_argument("--workload", default="c1", choices=("c1", "c3", "c4", "c5", "stream", "block", "probe-sweep"),
                    help="c1: the headline single-layer decode step, with c3, c5, stream and block sub-objects (default); "
                         "c3 / c4 / c5 alone: 40-layer stack of 128 tokens / batched decode of 64 Zipf-routed "
                         "tokens / 2048-token prefill on the grouped matrix-core path; stream: the streaming ceiling "
                         "of the c1 step's expert bytes (nmoe_hip_read_probe); block: the model's per-layer MoE "
                         "half (nmoe_moe_block); probe-sweep: the read ceiling against size and launch shape")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(expert parallelism is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import nmoe_hip as nh

    if args.timeline:
        if args.workload not in ("c1", "c3", "block", "c4", "c5"):
            raise SystemExit("--timeline: workloads c1, c3 and block (the fused launches), c4 and c5 (the grouped "
                             "GEMM launches)")
        nh.use_timeline_build()
        pool = Pool(nh, args, max_tokens=2048 if args.workload in ("c4", "c5") else 8)
        res = run_grouped(pool, args, args.workload) if args.workload in ("c4", "c5") else run_timeline(pool, args)
        print(json.dumps(res), flush=True)
        pool.ctx.close()
        return

    if args.copy_calib:
        ctx = nh.Context(0, max_tokens=1)
        n = args.copy_calib << 20
        src, dst = ctx.alloc(n, "calib.src"), ctx.alloc(n, "calib.dst")
        ev = HipEvents()
        for _ in range(5):
            ev.copy_d2d(dst.ptr, src.ptr, n, ctx.stream)
        ctx.sync()
        print(json.dumps({"copy_calib_bytes": n, "copies": 5}), flush=True)
        ctx.close()
        return

    if args.workload == "probe-sweep":
        print(json.dumps(run_probe_sweep(nh, args)), flush=True)
        return

    grouped = args.workload in ("c4", "c5") or (args.workload == "c1" and not args.no_extra)
    pool = Pool(nh, args, max_tokens=2048 if grouped else 8)
    if args.workload == "c3":
        result = run_c3(pool, args)
    elif args.workload == "stream":
        result = run_stream(pool, args)
    elif args.workload == "block":
        result = run_block(pool, args)
    elif args.workload in ("c4", "c5"):
        result = run_grouped(pool, args, args.workload)
    else:
        result = run_c1(pool, args)
        if not args.no_extra:
            print("[bench] c3, c4, c5, stream and block sub-benchmarks ...", file=sys.stderr, flush=True)
            result["c3"] = run_c3(pool, args)
            result["c4"] = run_grouped(pool, args, "c4")
            result["c5"] = run_grouped(pool, args, "c5")
            result["stream"] = run_stream(pool, args)
            result["block"] = run_block(pool, args)
        if not args.no_cpu:
            print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
            result["cpu_baseline"] = cpu_baseline(args.bits, args.k, args.seed, args.cpu_steps)
        if not args.no_extra and args.bits == 4:
            # the q2 configs on their own pool of 40 resident q2 layers (the q4 pool freed first)
            pool.ctx.close()
            a2 = argparse.Namespace(**vars(args))
            a2.bits = 2
            print("[bench] c2 (q2 top-8, top-6) and c5 q2 sub-benchmarks ...", file=sys.stderr, flush=True)
            pool = Pool(nh, a2, max_tokens=2048)
            result["c2"] = {}
            for k2 in (8, 6):
                a2.k = k2
                result["c2"][f"k{k2}"] = single_step_summary(run_c1(pool, a2), a2, cpu_steps=300)
            a2.k = 8
            result["c5_q2"] = run_grouped(pool, a2, "c5")
    pool.ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()

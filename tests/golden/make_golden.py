"""Writes tests/golden/math_ref_golden.npz from the reference's own CPU code.

Run in the build container (needs /root/reference): it loads
oracle/_ref/libnmoe_math_ref.so, which `make -C oracle ref` compiles from the
reference's src/math.m (as C, -O3 like the reference Makefile:7), and records
its outputs on crafted inputs.  Only the resulting vectors are committed.

Pure-math.m cases: softmax/top-k/renormalise (runtime.m:1498-1511 order),
RMSNorm, SiLU/sigmoid/SwiGLU, unpack/dequant rows, dequant matvec.
Composite cases ("step_*"): one decode token through a synthetic layer, with
the routing and every expert matvec/SwiGLU done by math.m and only the glue
(bf16 router dot products in the GPU's fixed order, the weighted combine of
kernels.metal:1394-1423) taken from the repository's oracle.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import binding as B  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "math_ref_golden.npz")


def ref_route(ref, logits: np.ndarray, k: int):
    """runtime.m:1498-1511 with math.m: softmax -> topk -> renormalize."""
    v = np.ascontiguousarray(logits, np.float32).copy()
    n = v.size
    ref.nmoe_cpu_softmax(v.ctypes.data, n)
    probs = v.copy()
    idx = np.zeros(B.MAX_K, np.uint64)
    val = np.zeros(B.MAX_K, np.float32)
    got = ref.nmoe_cpu_topk(v.ctypes.data, n, min(k, B.MAX_K), idx.ctypes.data, val.ctypes.data)
    ref.nmoe_cpu_renormalize(val.ctypes.data, got)
    idx8 = np.zeros(B.MAX_K, np.uint32)
    w8 = np.zeros(B.MAX_K, np.float32)
    idx8[:got] = idx[:got]
    w8[:got] = val[:got]
    return probs, idx8, w8, got


def route_cases(rng) -> list[tuple[np.ndarray, int]]:
    E = B.EXPERTS
    cases = []
    for i in range(16):  # plain N(0,1), k = 1..8
        cases.append((rng.standard_normal(E).astype(np.float32), 1 + i % 8))
    cases.append((np.zeros(E, np.float32), 8))  # all ties -> indices 0..7
    v = rng.standard_normal(E).astype(np.float32)
    v[[3, 200, 77, 150]] = 9.0  # planted exact ties at the top
    cases.append((v, 8))
    v = rng.standard_normal(E).astype(np.float32)
    v[[10, 11, 240]] = 5.0
    v[[5, 99]] = 4.0  # tie straddling the k boundary
    cases.append((v, 4))
    for _ in range(6):  # near ties: neighbours one ulp apart, so probabilities collide
        v = rng.standard_normal(E).astype(np.float32)
        top = np.argsort(-v)[:12]
        for j in range(0, 12, 2):
            v[top[j + 1]] = np.nextafter(v[top[j]], np.float32(-np.inf))
        cases.append((v, 8))
    for scale in (8.0, 20.0, 60.0):  # wide spread: terms below 2^-32 and underflow to 0
        cases.append(((rng.standard_normal(E) * scale).astype(np.float32), 8))
    v = rng.standard_normal(E).astype(np.float32)
    v[rng.choice(E, 40, replace=False)] = -np.inf
    cases.append((v, 8))
    v = np.full(E, -30.0, np.float32)  # many tiny equal terms + one dominant
    v[17] = 0.0
    v[200:] = np.linspace(-29, -31, 56, dtype=np.float32)
    cases.append((v, 8))
    # Zipf-skewed (batched-decode config) and uniform (prefill config) shapes
    ranks = rng.permutation(E) + 1
    g = -np.log(-np.log(rng.uniform(size=E)))
    cases.append(((-1.1 * np.log(ranks) + g).astype(np.float32), 8))
    cases.append((rng.uniform(size=E).astype(np.float32), 8))
    cases.append((rng.uniform(size=E).astype(np.float32), 6))
    return cases


def main():
    ref = B.ref_math()
    if ref is None:
        sys.exit("oracle/_ref/libnmoe_math_ref.so missing: run `make -C oracle ref` (needs /root/reference)")
    o = B.oracle()
    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}

    # ---- routing
    cases = route_cases(rng)
    L = np.stack([c[0] for c in cases])
    K = np.array([c[1] for c in cases], np.int32)
    P, I, W, N = [], [], [], []
    for lg, k in cases:
        probs, idx8, w8, got = ref_route(ref, lg, k)
        P.append(probs), I.append(idx8), W.append(w8), N.append(got)
    out.update(route_logits=L, route_k=K, route_probs=np.stack(P), route_idx=np.stack(I), route_w=np.stack(W),
               route_n=np.array(N, np.int32))
    # fewer experts than k (top-k clamps k to the count, math.m:103-105)
    small = rng.standard_normal(5).astype(np.float32)
    probs, idx8, w8, got = ref_route(ref, small, 8)
    out.update(small_logits=small, small_probs=probs, small_idx=idx8, small_w=w8, small_n=np.int32(got))

    # ---- RMSNorm (math.m:34-65)
    X = np.concatenate([rng.standard_normal((6, B.HIDDEN)), rng.standard_normal((2, B.HIDDEN)) * 1e-3,
                        rng.standard_normal((2, B.HIDDEN)) * 300.0]).astype(np.float32)
    Y = np.zeros_like(X)
    for i in range(X.shape[0]):
        ref.nmoe_cpu_rms_norm(X[i].ctypes.data, None, Y[i].ctypes.data, B.HIDDEN, C.c_float(1e-6), 0)
    wt = B.f32_to_bf16((rng.standard_normal(B.HIDDEN) * 0.1).astype(np.float32))
    Yw = np.zeros(B.HIDDEN, np.float32)
    ref.nmoe_cpu_rms_norm(X[0].ctypes.data, wt.ctypes.data, Yw.ctypes.data, B.HIDDEN, C.c_float(1e-6), 1)
    out.update(rms_x=X, rms_y=Y, rms_weight=wt, rms_y_weighted=Yw)

    # ---- SiLU / sigmoid / SwiGLU (math.m:21-32, 155-162)
    g = np.concatenate([rng.standard_normal(200) * 6, [0.0, -0.0, 88.0, -88.0, 1e-8, -1e-8]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    sw = np.zeros_like(g)
    ref.nmoe_cpu_swiglu(g.ctypes.data, u.ctypes.data, sw.ctypes.data, g.size)
    sig = np.array([ref.nmoe_cpu_sigmoid(float(v)) for v in g], np.float32)
    out.update(act_gate=g, act_up=u, act_swiglu=sw, act_sigmoid=sig)

    # ---- unpack / dequant rows / dequant matvec (math.m:191-274)
    for bits in (4, 2):
        ex = B.syn_expert(bits, 7, 3, 11, 0.02 if bits == 4 else 0.05)
        off = {4: (0, 524288, 557056, 1179648, 1703936, 1736704), 2: (0, 262144, 294912, 655360, 917504, 950272)}[bits]
        vpw = 32 // bits
        rows = 8
        wg = ex[off[0]:off[1]].view(np.uint32).reshape(512, 2048 // vpw)[:rows].copy()
        sg = ex[off[1]:off[2]].view(np.uint16).reshape(512, 32)[:rows].copy()
        bg = ex[off[2]:off[2] + 32768].view(np.uint16).reshape(512, 32)[:rows].copy()
        unp = np.zeros((rows, 2048), np.uint16)
        deq = np.zeros((rows, 2048), np.float32)
        for r in range(rows):
            ref.nmoe_cpu_unpack_row(wg[r].ctypes.data, unp[r].ctypes.data, 2048, bits)
            ref.nmoe_cpu_dequant_row(wg[r].ctypes.data, sg[r].ctypes.data, bg[r].ctypes.data, deq[r].ctypes.data,
                                     2048, bits)
        xv = rng.standard_normal(2048).astype(np.float32)
        mv = np.zeros(rows, np.float32)
        ref.nmoe_cpu_dequant_matvec(wg.ctypes.data, sg.ctypes.data, bg.ctypes.data, xv.ctypes.data, mv.ctypes.data,
                                    rows, 2048, bits)
        out.update({f"q{bits}_packed": wg, f"q{bits}_scales": sg, f"q{bits}_biases": bg, f"q{bits}_unpacked": unp,
                    f"q{bits}_dequant": deq, f"q{bits}_x": xv, f"q{bits}_matvec": mv})

    # ---- composite decode steps on the synthetic configs
    for name, bits, k, sigma in (("step_q4_k8", 4, 8, 0.02), ("step_q2_k8", 2, 8, 0.05), ("step_q2_k6", 2, 6, 0.05)):
        seed, layer = 0, 0
        router = B.syn_bf16(B.EXPERTS * B.HIDDEN, seed, layer, 16, 0.02).reshape(B.EXPERTS, B.HIDDEN)
        x = B.bf16_to_f32(B.syn_bf16(B.HIDDEN, seed, layer, 17, 1.0))
        h_mid = B.bf16_to_f32(B.syn_bf16(B.HIDDEN, seed, layer, 18, 1.0))
        logits = B.router_logits_bf16(router, x)
        _, idx8, w8, got = ref_route(ref, logits, k)
        ys = np.zeros((got, B.HIDDEN), np.float32)
        for s in range(got):
            ex = B.syn_expert(bits, seed, layer, int(idx8[s]), sigma)
            off = B.EXPERT_SIZE[bits]
            o9 = {4: (0, 524288, 557056, 589824, 1114112, 1146880, 1179648, 1703936, 1736704),
                  2: (0, 262144, 294912, 327680, 589824, 622592, 655360, 917504, 950272)}[bits]
            gate = np.zeros(512, np.float32)
            up = np.zeros(512, np.float32)
            act = np.zeros(512, np.float32)
            base = ex.ctypes.data
            ref.nmoe_cpu_dequant_matvec(base + o9[0], base + o9[1], base + o9[2], x.ctypes.data, gate.ctypes.data,
                                        512, 2048, bits)
            ref.nmoe_cpu_dequant_matvec(base + o9[3], base + o9[4], base + o9[5], x.ctypes.data, up.ctypes.data,
                                        512, 2048, bits)
            ref.nmoe_cpu_swiglu(gate.ctypes.data, up.ctypes.data, act.ctypes.data, 512)
            ref.nmoe_cpu_dequant_matvec(base + o9[6], base + o9[7], base + o9[8], act.ctypes.data, ys[s].ctypes.data,
                                        2048, 512, bits)
            del off
        res = np.zeros(B.HIDDEN, np.float32)
        o.orc_combine(h_mid.ctypes.data, ys.ctypes.data, w8.ctypes.data, got, None, None, res.ctypes.data, B.HIDDEN)
        out.update({f"{name}_logits": logits, f"{name}_idx": idx8, f"{name}_w": w8, f"{name}_out": res})

    # ---- fp32 -> bf16 (math.m:14-19) on raw bit patterns: rounding ties both
    # ways, carries into the exponent, subnormals, the largest finite values
    # (which round to Inf), infinities and NaN payloads (which the reference's
    # carry can turn into Inf or wrap to zero), then uniform random patterns
    # (their own generator, so the arrays above keep their values).
    crafted = [0x00000000, 0x80000000, 0x3F800000, 0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF, 0x3F818001,
               0x3FFF8000, 0x3FFFFFFF, 0x00000001, 0x00008000, 0x00018000, 0x00017FFF, 0x007FFFFF, 0x00800000,
               0x80008000, 0x80018000, 0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0xFF7F8000, 0x7F800000, 0xFF800000,
               0x7FC00000, 0x7F800001, 0x7F808000, 0x7FBFFFFF, 0x7FFF8000, 0x7FFFFFFF, 0xFFC00000, 0xFFFF8000,
               0xFFFFFFFF, 0x40490FDB, 0xC2F6E979, 0x33D6BF95]
    rb = np.random.default_rng(20261202)
    bits_in = np.concatenate([np.array(crafted, np.uint32),
                              rb.integers(0, 2**32, size=4096, dtype=np.uint64).astype(np.uint32)])
    bf_out = np.zeros(bits_in.size, np.uint16)
    ref.orc_ref_f32_to_bf16_bits(bits_in.ctypes.data, bf_out.ctypes.data, bits_in.size)
    out.update(f2bf_in=bits_in, f2bf_out=bf_out)

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()

"""C3 at its configuration: the routed-expert stack of 128 sequential decode
tokens through 40 resident q4 layers (40 x 453 MB = 18.1 GB in HBM), each
with its own bf16 router, h_{l+1} = h_l + MoE_l(RMSNorm(h_l)) -- the layer
loop of NMOEProcessToken (src/runtime.m:3732-3777) restricted to its MoE
tails.

Checked, layer by layer on the GPU's own inputs (teacher-forced):
  - every token's routing at every layer bit-exact with the oracle
    (RMSNorm math.m:34-65, router, softmax/top-k/renormalise math.m:67-153):
    128 x 40 routings;
  - every token's 41 hidden states, 40 routings and weights bit for bit
    against the one-launch-per-layer form (the fused single-layer launch,
    which the oracle pins on its own);
  - every token's 40 layer outputs within
    max-abs 2e-3 / rel-L2 1e-3 of the oracle's layer (orc_moe_layer_rmsnorm);
  - every hidden state finite and the device status clean."""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import assert_close
from oracle import binding as B

pytestmark = pytest.mark.gpu

NL, NTOK, K, SEED, SIGMA = 40, 128, 8, 0, 0.02


def _oracle_layer(pack, W, h_in):
    h_out = np.zeros(2048, np.float32)
    idx, w = np.zeros(8, np.uint32), np.zeros(8, np.float32)
    rc = B.oracle().orc_moe_layer_rmsnorm(pack.ctypes.data, 4, W.ctypes.data,
                                          np.ascontiguousarray(h_in, np.float32).ctypes.data, 1e-6, K,
                                          h_out.ctypes.data, idx.ctypes.data, w.ctypes.data, None)
    assert rc == 0
    return h_out, idx, w


def test_stack_40_layers_128_tokens():
    import nmoe_hip as nh
    with nh.Context(0, max_tokens=4) as ctx:
        print(f"[c3] making {NL} q4 layers resident", flush=True)
        for layer in range(NL):
            ctx.synth_layer(layer, 4, SEED, SIGMA)
        W = [np.ascontiguousarray(B.syn_bf16(256 * 2048, SEED, layer, 16, 0.02).reshape(256, 2048))
             for layer in range(NL)]
        routers_dev = ctx.alloc(NL * 256 * 2048 * 2)
        for layer in range(NL):
            routers_dev.upload(W[layer], offset=layer * 256 * 2048 * 2)
        routers = [ctx.router_bf16(routers_dev.ptr + layer * 256 * 2048 * 2) for layer in range(NL)]
        H0 = np.stack([B.bf16_to_f32(B.syn_bf16(2048, SEED, 99, 1000 + t, 1.0)) for t in range(NTOK)])
        hs, idx_s, w_s = ctx.alloc((NL + 1) * 8192), ctx.alloc(NL * 32), ctx.alloc(NL * 32)
        HS, IS, WS = [], [], []
        for t in range(NTOK):
            hs.upload(H0[t])
            ctx._check(ctx.moe_stack(list(range(NL)), routers, K, 1e-6, hs, idx_s, w_s))
            HS.append(hs.download(np.float32, (NL + 1, 2048)))
            IS.append(idx_s.download(np.uint32, (NL, 8)))
            WS.append(w_s.download(np.float32, (NL, 8)))
        assert ctx.device_status() == nh.OK
        print("[c3] every token again, one launch per layer", flush=True)
        try:
            ctx._check(ctx.set_option(nh.OPT_STACK_LOOP, 0))
            for t in range(NTOK):
                hs.upload(H0[t])
                ctx._check(ctx.moe_stack(list(range(NL)), routers, K, 1e-6, hs, idx_s, w_s))
                np.testing.assert_array_equal(hs.download(np.float32, (NL + 1, 2048)).view(np.uint32),
                                              HS[t].view(np.uint32), err_msg=f"token {t} hidden states")
                np.testing.assert_array_equal(idx_s.download(np.uint32, (NL, 8)), IS[t], err_msg=f"token {t}")
                np.testing.assert_array_equal(w_s.download(np.float32, (NL, 8)).view(np.uint32),
                                              WS[t].view(np.uint32), err_msg=f"token {t} weights")
        finally:
            ctx._check(ctx.set_option(nh.OPT_STACK_LOOP, 1))
        assert ctx.device_status() == nh.OK
    print("[c3] checking routing of every token at every layer", flush=True)
    x = np.zeros(2048, np.float32)
    o = B.oracle()
    for t in range(NTOK):
        H = HS[t]
        assert np.isfinite(H).all(), f"token {t}"
        np.testing.assert_array_equal(H[0], H0[t])
        for l in range(NL):
            o.orc_rms_norm(np.ascontiguousarray(H[l]).ctypes.data, None, x.ctypes.data, 2048, 1e-6, 0)
            oi, ow, _ = B.route(B.router_logits_bf16(W[l], x), K)
            np.testing.assert_array_equal(IS[t][l], oi, err_msg=f"token {t} layer {l}")
            np.testing.assert_array_equal(WS[t][l].view(np.uint32), ow.view(np.uint32), err_msg=f"token {t} layer {l}")
    esz = B.EXPERT_SIZE[4]

    def check_token(t):  # the C calls release the interpreter lock
        for l in range(NL):
            pack = np.zeros(256 * esz, np.uint8)
            for e in IS[t][l]:
                pack[int(e) * esz:(int(e) + 1) * esz] = B.syn_expert(4, SEED, l, int(e), SIGMA)
            want, oi, ow = _oracle_layer(pack, W[l], HS[t][l])
            np.testing.assert_array_equal(oi, IS[t][l])
            assert_close(HS[t][l + 1], want, what=f"token {t} layer {l}")

    tokens = list(range(NTOK))
    print(f"[c3] {len(tokens)} tokens: 40 layer outputs each against the oracle", flush=True)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        list(ex.map(check_token, tokens))

"""FP8 (128x128 block e4m3) and MXFP4 expert weights in the fused decode MoE
on the GPU vs the oracle.

Packers bit-exact (the MXFP4 quantizer against oracle/mx.py's OCP
restatement, the FP8 codes against quantize_fp8_block, both tile layouts
against their restated packers); the MoE output within max-abs-rel 1e-2 of
the fp32 oracle evaluated on the oracle's own quantization of the same
weights (its only deviations are the fp16 activations and fp16 h; MXFP4
codes enter the MFMAs as fp16(code x scale), exact at these weights' block
scales, all >= 2^-14).
"""
import numpy as np
import pytest

from oracle import moe as OM
from oracle import mx
from oracle import quant as Q

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _weights(rng, E, out_f, in_f, scale=0.05):
    return (rng.standard_normal((E, out_f, in_f)) * scale).astype(np.float16).astype(np.float32)


def _oracle_deq(fmt, W):
    """Oracle quantization of W (E, out, in) and its dequantized weights."""
    E, out_f, in_f = W.shape
    flat = W.reshape(E * out_f, in_f)
    if fmt == "fp8":
        q, s = Q.quantize_fp8_block(flat)
        return Q.dequantize_fp8_block(q, s).reshape(E, out_f, in_f)
    p, e8 = mx.quantize_mxfp4(flat)
    return mx.dequantize_mxfp4(p, e8).reshape(E, out_f, in_f)


def _layer(rng, fmt, E, hidden, inter, sinter):
    from fastllm_py.kernels import moe_int4

    Wr = {"gate": _weights(rng, E, inter, hidden), "up": _weights(rng, E, inter, hidden),
          "down": _weights(rng, E, hidden, inter)}
    st = {"group": moe_int4.LOWP_FORMATS[fmt][1], "format": fmt}
    for p, w in Wr.items():
        st.update(moe_int4.stack_lowp(fmt, p, w))
    deq = {p: _oracle_deq(fmt, w) for p, w in Wr.items()}
    sh = sdeq = None
    if sinter:
        Ws = {"gate": _weights(rng, 1, sinter, hidden), "up": _weights(rng, 1, sinter, hidden),
              "down": _weights(rng, 1, hidden, sinter)}
        sh = {"group": st["group"], "format": fmt}
        for p, w in Ws.items():
            sh.update(moe_int4.stack_lowp(fmt, p, w))
        sdeq = {p: _oracle_deq(fmt, w) for p, w in Ws.items()}
    return st, deq, sh, sdeq


def test_mxfp4_quantizer_bit_exact(torch_gpu):
    from fastllm_py import quantizer

    rng = np.random.default_rng(11)
    w = (rng.standard_normal((96, 512)) * 0.03).astype(np.float32)
    w[0, :32] = 0.0                                   # all-zero block
    w[1, :32] = -0.0
    w[2, :32] = np.float32(2.0 ** -140)               # subnormal block
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 7.9], np.float32)
    w[3, :32] = 0.0
    w[3, 0] = 6.0                                     # X = 1: the rest are exact midpoints
    w[3, 1:10] = mids
    w[3, 10:19] = -mids
    w[4, :64] = rng.uniform(-3e4, 3e4, 64).astype(np.float32)
    qt = quantizer.quantize_mxfp4(w)
    p, e8 = mx.quantize_mxfp4(w)
    np.testing.assert_array_equal(qt.data, p)
    np.testing.assert_array_equal(qt.scales, e8)
    np.testing.assert_array_equal(quantizer.dequantize_mxfp4(qt).view(np.uint32),
                                  mx.dequantize_mxfp4(p, e8).view(np.uint32))


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_lowp_tiles_bit_exact(torch_gpu, fmt):
    from fastllm_py.kernels import moe_int4

    rng = np.random.default_rng(12)
    E, out_f, in_f = 3, 256, 384
    W = _weights(rng, E, out_f, in_f)
    st = moe_int4.stack_lowp(fmt, "gate", W)
    flat = W.reshape(E * out_f, in_f)
    if fmt == "fp8":
        q, s = Q.quantize_fp8_block(flat)
        want_q, want_s = mx.moe_tile_pack_fp8(q), s
    else:
        p, e8 = mx.quantize_mxfp4(flat)
        want_q, want_s = mx.moe_tile_pack_mxfp4(p, e8)
        want_s = want_s.view(np.int32)
    got_q = st["gate.qtile"].cpu().numpy().reshape(want_q.shape)
    got_s = st["gate.sz"].cpu().numpy().reshape(want_s.shape)
    np.testing.assert_array_equal(got_q, want_q)
    np.testing.assert_array_equal(got_s.view(np.uint32), want_s.view(np.uint32))


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
@pytest.mark.parametrize("T,E,K,hidden,inter,sinter", [
    (1, 16, 4, 1024, 512, 1024),
    (3, 16, 4, 1024, 512, 1024),
    (8, 12, 4, 512, 768, 0),
    (16, 16, 4, 1024, 512, 1536),
])
def test_lowp_moe_parity(torch_gpu, fmt, T, E, K, hidden, inter, sinter):
    """Router + fused MoE (moe_route_forward) and the list-driven call
    (moe_forward) with FP8 / MXFP4 experts vs the fp32 oracle; routing is the
    INT4 path's (bit-exact, tested there), so the oracle takes the router's
    picks."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(1300 + T * 7 + hidden + (0 if fmt == "fp8" else 1))
    st, deq, sh, sdeq = _layer(rng, fmt, E, hidden, inter, sinter)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda() if sinter else None
    ref_r = route_topk_device(logits, K, shared_logit=sl)
    ids, w = ref_r["topk_ids"].cpu().numpy(), ref_r["topk_w"].cpu().numpy()
    coef = 1.0 / (1.0 + np.exp(-sl.cpu().numpy())) if sinter else None
    ref = OM.moe_ref(x.cpu().numpy(), deq, ids, w, sdeq, coef)
    for call in range(2):
        r = {}
        y = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, shared=sh,
                                       shared_inter=sinter, shared_logit=sl, route=r)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(r["topk_ids"].cpu().numpy(), ids)
        err = Q.max_abs_rel(y.cpu().numpy(), ref)
        assert err < TOL, (fmt, call, err)
    y2 = moe_int4.moe_forward(x, st, E, hidden, inter, ref_r, max_slots=min(E, T * K),
                              max_entries=T * K, shared=sh, shared_inter=sinter,
                              shared_coef=ref_r.get("shared_coef"))
    assert Q.max_abs_rel(y2.cpu().numpy(), ref) < TOL


_C4 = {}  # fmt -> (weights, stacks, per-expert oracle dequantization cache)


def _config4_layer(torch, fmt):
    """Qwen1.5-MoE-A2.7B expert weights in `fmt`, built once per format."""
    from fastllm_py.kernels import moe_int4

    if fmt not in _C4:
        E, hidden, inter, sinter = 60, 2048, 1408, 5632
        rng = np.random.default_rng(1400 + (0 if fmt == "fp8" else 1))

        def w(n, o, i):
            return (rng.standard_normal((n, o, i), dtype=np.float32) * 0.05
                    ).astype(np.float16).astype(np.float32)
        Wr = {"gate": w(E, inter, hidden), "up": w(E, inter, hidden), "down": w(E, hidden, inter)}
        Ws = {"gate": w(1, sinter, hidden), "up": w(1, sinter, hidden), "down": w(1, hidden, sinter)}
        st = {"group": moe_int4.LOWP_FORMATS[fmt][1], "format": fmt}
        sh = dict(st)
        for p in ("gate", "up", "down"):
            st.update(moe_int4.stack_lowp(fmt, p, Wr[p]))
            sh.update(moe_int4.stack_lowp(fmt, p, Ws[p]))
        sdeq = {p: _oracle_deq(fmt, Ws[p]) for p in Ws}
        torch.cuda.synchronize()
        _C4[fmt] = (Wr, st, sh, sdeq, {})
    return _C4[fmt]


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
@pytest.mark.parametrize("T", [1, 6, 16])
def test_lowp_moe_config4_shape(torch_gpu, fmt, T):
    """Qwen1.5-MoE-A2.7B shapes (60 experts, hidden 2048, inter 1408, shared
    5632) at 1, 6 and 16 tokens -- the launch shapes the decode plan picks
    there (at 16 tokens: four gate/up tiles and two blocks per wave) -- twice
    in a row: the oracle dequantizes only the routed experts (the blocks of
    one expert depend on that expert's weights alone)."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    E, K, hidden, inter, sinter = 60, 4, 2048, 1408, 5632
    Wr, st, sh, sdeq, cache = _config4_layer(torch, fmt)
    rng = np.random.default_rng(1410 + T + (0 if fmt == "fp8" else 100))
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda()
    coef = 1.0 / (1.0 + np.exp(-sl.cpu().numpy()))
    ref = None
    for call in range(2):
        r = {}
        print(f"lowp config4 {fmt} T={T} call {call}", flush=True)
        y = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, shared=sh,
                                       shared_inter=sinter, shared_logit=sl, route=r)
        torch.cuda.synchronize()
        if ref is None:
            ids, w = r["topk_ids"].cpu().numpy(), r["topk_w"].cpu().numpy()
            deq = {p: np.zeros((E,) + Wr[p].shape[1:], np.float32) for p in Wr}
            for e in sorted(set(ids.reshape(-1).tolist())):
                if e not in cache:
                    cache[e] = {p: _oracle_deq(fmt, Wr[p][e:e + 1])[0] for p in Wr}
                for p in Wr:
                    deq[p][e] = cache[e][p]
            ref = OM.moe_ref(x.cpu().numpy(), deq, ids, w, sdeq, coef)
        else:
            np.testing.assert_array_equal(r["topk_ids"].cpu().numpy(), ids)
        err = Q.max_abs_rel(y.cpu().numpy(), ref)
        assert err < TOL, (fmt, T, call, err)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
@pytest.mark.parametrize("T,E,K,hidden,inter,sinter,norm", [
    (40, 16, 4, 1024, 512, 1024, False),
    (200, 32, 8, 512, 768, 0, True),
    (130, 8, 2, 256, 256, 512, False),
])
def test_lowp_moe_prefill_parity(torch_gpu, fmt, T, E, K, hidden, inter, sinter, norm):
    """More than 16 tokens: the grouped MFMA kernels with FP8 / MXFP4 experts
    (router lists from route_topk_device) vs the fp32 oracle, and the routed
    entry (moe_route_forward: lists built in the router launch) against
    them."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(1500 + T + E + (0 if fmt == "fp8" else 1))
    st, deq, sh, sdeq = _layer(rng, fmt, E, hidden, inter, sinter)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda() if sinter else None
    r = route_topk_device(logits, K, norm_topk_prob=norm, shared_logit=sl)
    ids, w = r["topk_ids"].cpu().numpy(), r["topk_w"].cpu().numpy()
    coef = 1.0 / (1.0 + np.exp(-sl.cpu().numpy())) if sinter else None
    ref = OM.moe_ref(x.cpu().numpy(), deq, ids, w, sdeq, coef)
    y = moe_int4.moe_forward(x, st, E, hidden, inter, r, max_slots=E, max_entries=T * K, shared=sh,
                             shared_inter=sinter, shared_coef=r.get("shared_coef"))
    torch.cuda.synchronize()
    assert Q.max_abs_rel(y.cpu().numpy(), ref) < TOL, fmt
    # the one-call routed entry: the same picks, y up to the atomic order
    o = {}
    y2 = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, norm_topk_prob=norm,
                                    shared=sh, shared_inter=sinter, shared_logit=sl, route=o)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(o["topk_ids"].cpu().numpy(), ids)
    assert Q.max_abs_rel(y2.cpu().numpy(), y.cpu().numpy()) < 1e-6, fmt


def test_lowp_rejects(torch_gpu):
    """A wrong group size or mixed formats are refused before any launch."""
    from fastllm_py import _native
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(15)
    st, _, _, _ = _layer(rng, "fp8", 4, 256, 256, 0)
    x = torch.zeros((1, 256), device="cuda")
    int4_sh = moe_int4.build_stacked_experts(
        [{"gate": np.zeros((256, 256), np.float16), "up": np.zeros((256, 256), np.float16),
          "down": np.zeros((256, 256), np.float16)}], 128)
    L1 = moe_int4.build_lists(1, 4, rw=torch.full((1, 4), 0.25, device="cuda"))
    with pytest.raises(ValueError):
        moe_int4.moe_forward(x, st, 4, 256, 256, L1, shared=int4_sh, shared_inter=256)
    lib = _native.lib()
    p = 1 << 20  # never dereferenced: the checks fail first
    ws = moe_int4.moe_workspace_bytes(1, 256, 256, 0, 4)
    args = lambda gs: [p, 1, 256, gs, 4, 256] + [p] * 6 + [0] + [None] * 6 + [None] + [p] * 5 + \
        [4, 4, p, ws, p, None]  # noqa: E731
    assert lib.fastllm_moe_lowp_fused(1, *args(32)) == 1   # FP8 takes group 128
    assert lib.fastllm_moe_lowp_fused(2, *args(128)) == 1  # MXFP4 takes group 32
    assert lib.fastllm_moe_lowp_fused(0, *args(128)) == 1  # INT4 goes through its own entry
    assert lib.fastllm_moe_lowp_fused(3, *args(128)) == 1

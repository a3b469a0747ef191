"""Row-major INT4 GEMV, gate matvec, router and fused MoE on the GPU vs the oracle.

Mirrors tests/test_moe_int4.py of the reference (same shapes and seeds where
it has them) with the bar of this build: packers and routing bit-exact,
matmul paths within max-abs-rel 1e-2 (tighter bounds asserted where the
kernel's only deviation is fp16 activation rounding).
"""
import os

import numpy as np
import pytest

from oracle import moe as OM
from oracle import quant as Q
from oracle import router as R

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _experts(rng, E, hidden, inter, scale=0.1):
    return [{"gate": (rng.standard_normal((inter, hidden)) * scale).astype(np.float16),
             "up": (rng.standard_normal((inter, hidden)) * scale).astype(np.float16),
             "down": (rng.standard_normal((hidden, inter)) * scale).astype(np.float16)}
            for _ in range(E)]


def _stacked(experts, gs):
    """The product's stacked experts, and the oracle's own row-major
    quantization (quantize_int4_rowmajor restated in oracle/quant.py) of the
    same fp16 weights -- what the oracle dequantizes.  The product's tile
    pack of those bytes is pinned separately (test_moe_tile_pack_bit_exact)."""
    from fastllm_py.kernels import moe_int4

    st = moe_int4.build_stacked_experts(experts, gs)
    orc = {}
    for proj in ("gate", "up", "down"):
        p, s_, z = Q.quantize_int4_rowmajor(np.stack([e[proj] for e in experts]), gs)
        orc.update({f"{proj}.qweight": p, f"{proj}.scales": s_, f"{proj}.zeros": z})
    return st, orc


def _np_stacked(st):
    """Tile-layout stacked experts -> row-major numpy arrays for the oracle."""
    from fastllm_py.kernels import moe_int4

    return {k: (v.cpu().numpy() if hasattr(v, "cpu") else v)
            for k, v in moe_int4.unpack_stacked(st).items()}


# ------------------------------------------------------------ row-major packers
def test_rowmajor_quantize_bit_exact_and_batched(torch_gpu):
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((3, 96, 384)) * 0.1).astype(np.float16)
    W[1, 5, :128] = 0.25
    for gs in (128, 32):
        pb, sb, zb = Q.quantize_int4_rowmajor(W, gs)
        qw, sc, ze, shp = moe_int4._quantize_int4_rowmajor_batched(torch.from_numpy(W).cuda(), gs)
        np.testing.assert_array_equal(qw.cpu().numpy(), pb)
        np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint16), sb.view(np.uint16))
        np.testing.assert_array_equal(ze.cpu().numpy().view(np.uint16), zb.view(np.uint16))
        pay = moe_int4.quantize_int4_rowmajor(W[2], gs)  # numpy in -> numpy out
        np.testing.assert_array_equal(pay["qweight"], pb[2])
        np.testing.assert_array_equal(moe_int4.dequantize_int4_rowmajor(pay),
                                      Q.dequantize_int4_rowmajor(pb[2], sb[2], zb[2], gs))


def test_packer_golden_fixture(torch_gpu):
    from fastllm_py import quantizer
    from fastllm_py.kernels import marlin, moe_int4
    from fastllm_py.moe import _quantize_marlin_device

    torch = torch_gpu
    g = np.load(os.path.join(GOLDEN, "packers.npz"))
    w = g["w"]
    qt = quantizer.quantize_int4_group(w, 128)
    np.testing.assert_array_equal(qt.data, g["group_packed"])
    np.testing.assert_array_equal(qt.scales, g["group_scales"])
    np.testing.assert_array_equal(qt.zeros, g["group_zeros"])
    q, s, z = _quantize_marlin_device(torch.from_numpy(w).cuda(), 128)
    np.testing.assert_array_equal(q.cpu().numpy(), g["marlin_q"])
    np.testing.assert_array_equal(marlin.pack_gptq_qweight(q.cpu().numpy()), g["marlin_gptq"])
    s16, zp = marlin.build_marlin_scales_zeros(s.cpu().numpy(), z.cpu().numpy(), 128)
    np.testing.assert_array_equal(s16, g["marlin_scales"])
    np.testing.assert_array_equal(zp, g["marlin_zeros"])
    pay = moe_int4.quantize_int4_rowmajor(w.astype(np.float16), 128)
    np.testing.assert_array_equal(pay["qweight"], g["rowmajor_packed"])
    np.testing.assert_array_equal(pay["scales"], g["rowmajor_scales"])
    np.testing.assert_array_equal(pay["zeros"], g["rowmajor_zeros"])
    f8 = quantizer.quantize_fp8_block(g["fp8_w"], 128)
    np.testing.assert_array_equal(f8.data, g["fp8_q"])
    np.testing.assert_array_equal(f8.scales, g["fp8_scales"])


def test_moe_tile_pack_bit_exact(torch_gpu):
    """GPU tile repack equals the oracle's layout; unpack inverts it exactly;
    build_stacked_experts stores exactly the tile pack of the row-major
    quantization."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(6)
    for E, out_f, in_f, gs in [(3, 48, 256, 128), (2, 32, 384, 32), (1, 16, 128, 64)]:
        W = (rng.standard_normal((E, out_f, in_f)) * 0.1).astype(np.float16)
        pb, sb, zb = Q.quantize_int4_rowmajor(W, gs)
        qt, sz = moe_int4.tile_pack(torch.from_numpy(pb).cuda(), torch.from_numpy(sb).cuda(),
                                    torch.from_numpy(zb).cuda(), gs)
        oq, osz = Q.moe_tile_pack(pb.reshape(E * out_f, -1), sb.reshape(E * out_f, -1),
                                  zb.reshape(E * out_f, -1))
        np.testing.assert_array_equal(qt.cpu().numpy(), oq)
        np.testing.assert_array_equal(sz.cpu().numpy().view(np.uint32), osz)
        q2, s2, z2 = moe_int4.tile_unpack(qt, sz, E * out_f, in_f, gs)
        np.testing.assert_array_equal(q2.cpu().numpy(), pb.reshape(E * out_f, -1))
        np.testing.assert_array_equal(s2.cpu().numpy().view(np.uint16), sb.reshape(E * out_f, -1).view(np.uint16))
        np.testing.assert_array_equal(z2.cpu().numpy().view(np.uint16), zb.reshape(E * out_f, -1).view(np.uint16))
    ex = _experts(rng, 2, 256, 128)
    st = moe_int4.build_stacked_experts(ex, 64)
    rm = _np_stacked(st)
    for proj in ("gate", "up", "down"):
        pb, sb, zb = Q.quantize_int4_rowmajor(np.stack([e[proj] for e in ex]), 64)
        np.testing.assert_array_equal(rm[f"{proj}.qweight"], pb)
        np.testing.assert_array_equal(rm[f"{proj}.scales"].view(np.uint16), sb.view(np.uint16))
        np.testing.assert_array_equal(rm[f"{proj}.zeros"].view(np.uint16), zb.view(np.uint16))


# ------------------------------------------------------------------- GEMVs
@pytest.mark.parametrize("out_f,in_f,gs", [(1408, 2048, 128), (2048, 1408, 128), (512, 1024, 128),
                                           (256, 256, 32), (4096, 4096, 128), (200, 512, 64)])
def test_gemv_int4_matches_dequant(torch_gpu, out_f, in_f, gs):
    # reference tests/test_moe_int4.py:10-20
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((out_f, in_f)) * 0.1).astype(np.float32)
    x = (rng.standard_normal(in_f) * 0.5).astype(np.float32)
    payload = moe_int4.quantize_int4_rowmajor(torch.from_numpy(w).cuda(), gs)
    y = moe_int4.gemv_int4(torch.from_numpy(x).cuda(), payload).cpu().numpy()
    p, s, z = Q.quantize_int4_rowmajor(w, gs)
    ref = x @ Q.dequantize_int4_rowmajor(p, s, z, gs).T
    assert y.shape == (out_f,)
    assert Q.max_abs_rel(y, ref) < 2e-3


@pytest.mark.parametrize("M", [1, 4, 16, 20])
def test_dgemv_fp16_batched(torch_gpu, M):
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(M)
    out_f, in_f = 1024, 4096
    w = (rng.standard_normal((out_f, in_f)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, in_f)).astype(np.float16)
    payload = moe_int4.quantize_int4_rowmajor(torch.from_numpy(w).cuda(), 128)
    if M == 1:
        y = moe_int4.dgemv(torch.from_numpy(x).cuda(), payload)
        assert y.shape == (1, out_f) and y.dtype == torch.float16
    else:
        y = moe_int4._rm_gemv(torch.from_numpy(x).cuda(), payload, None, torch.float16)
    p, s, z = Q.quantize_int4_rowmajor(w, 128)
    ref = x.astype(np.float32) @ Q.dequantize_int4_rowmajor(p, s, z, 128).T
    assert Q.max_abs_rel(y.float().cpu().numpy(), ref) < 2e-3


RM_LINE_CASES = [
    # (out, in, M, x dtype, y dtype): the whole-line kernel (M <= 4, in % 256 == 0)
    (6144, 4096, 1, "f16", "f16"),   # Qwen3-8B qkv: two tiles per workgroup
    (4096, 12288, 1, "f16", "f16"),  # down: three pairs per wave
    (4096, 12288, 2, "f32", "f32"),  # fp32 rows, one copy per block
    (6144, 4096, 3, "f32", "f16"),   # fp32 rows, two copies per block
    (1000, 1536, 4, "f16", "f32"),   # ragged N, 6 pairs on 8 waves
    (17, 768, 2, "f16", "f16"),      # N < one tile
    (64, 16384, 1, "f32", "f32"),    # four pairs per wave
    (2048, 1408, 1, "f16", "f16"),   # in % 256 == 128: the tile kernel
]


@pytest.mark.parametrize("out_f,in_f,M,xd,yd", RM_LINE_CASES)
def test_rowmajor_gemv_shapes(torch_gpu, out_f, in_f, M, xd, yd):
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    dt = {"f16": torch.float16, "f32": torch.float32}
    rng = np.random.default_rng(out_f + in_f + M)
    w = (rng.standard_normal((out_f, in_f)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, in_f)).astype(np.float32)
    payload = moe_int4.quantize_int4_rowmajor(torch.from_numpy(w).cuda(), 128)
    xg = torch.from_numpy(x).cuda().to(dt[xd])
    y = moe_int4._rm_gemv(xg, payload, None, dt[yd])
    assert y.shape == (M, out_f) and y.dtype == dt[yd]
    p, s, z = Q.quantize_int4_rowmajor(w, 128)
    ref = xg.float().cpu().numpy() @ Q.dequantize_int4_rowmajor(p, s, z, 128).T
    assert Q.max_abs_rel(y.float().cpu().numpy(), ref) < 2e-3


def test_gate_matvec(torch_gpu):
    # reference tests/test_moe_int4.py:57-64
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(3)
    E, hidden = 60, 2048
    gw = (rng.standard_normal((E, hidden)) * 0.1).astype(np.float16)
    x = (rng.standard_normal(hidden) * 0.3).astype(np.float32)
    y = moe_int4.gate_matvec(torch.from_numpy(x).cuda(), torch.from_numpy(gw).cuda(), E, hidden)
    ref = x @ gw.astype(np.float32).T
    np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------ router
@pytest.mark.parametrize("name", ["qwen15moe_t1", "qwen15moe_t16", "qwen3moe_t512", "deepseek_t32",
                                  "ties_e60_k4", "ties_e128_k8", "ties_e256_k16", "ties_groups"])
def test_route_golden(torch_gpu, name):
    """Bit-exact against the reference's selection on every token, tied ones
    included: the fixtures hold np.argpartition's own choice and order
    (expert_router.py:50,55), taken on the generating host, and the ties_*
    fixtures hold 42-95 tokens with experts tied at the k-th value."""
    from fastllm_py.expert_router import route_topk, route_topk_device

    g = np.load(os.path.join(GOLDEN, f"route_{name}.npz"))
    logits = g["logits"]
    kw = dict(norm_topk_prob=bool(g["norm"]), scoring=str(g["scoring"]),
              routed_scaling=float(g["scale"]), e_score_bias=g["bias"] if g["bias"].size else None,
              n_group=int(g["n_group"]), topk_group=int(g["topk_group"]))
    k = int(g["top_k"])
    r = route_topk_device(logits, k, **kw)
    ids = r["topk_ids"].cpu().numpy()
    w = r["topk_w"].cpu().numpy()
    np.testing.assert_array_equal(ids, g["idx_argpartition"])
    np.testing.assert_array_equal(w.view(np.uint32), g["w_argpartition"].view(np.uint32))
    if name.startswith("ties"):
        assert int(g["boundary_ties"].sum()) >= 20
    # ExpertTask lists equal the oracle's (restated argpartition)
    tasks = route_topk(logits, k, **kw)
    ref_tasks = R.route_topk(logits.astype(np.float32), k, **kw)
    assert R.tasks_to_dict(tasks) == R.tasks_to_dict(ref_tasks)


def test_route_random_live_oracle(torch_gpu):
    from fastllm_py.expert_router import route_topk_device

    rng = np.random.default_rng(99)
    for T, E, k, norm in [(7, 60, 4, False), (33, 128, 8, True), (16, 256, 16, True), (3, 8, 2, False)]:
        s = (rng.standard_normal((T, E)) * 3).astype(np.float32)
        r = route_topk_device(s, k, norm_topk_prob=norm, routed_scaling=1.5)
        _, ic, wc = R.route_topk(s, k, norm_topk_prob=norm, routed_scaling=1.5,
                                 return_arrays=True)
        np.testing.assert_array_equal(r["topk_ids"].cpu().numpy(), ic)
        np.testing.assert_array_equal(r["topk_w"].cpu().numpy().view(np.uint32), wc.view(np.uint32))
        rw = r["rw"].cpu().numpy()
        dense = np.zeros((T, E), np.float32)
        np.put_along_axis(dense, ic, wc, axis=-1)
        np.testing.assert_array_equal(rw, dense)


@pytest.mark.parametrize("E", [8, 16, 60, 64, 128, 256])
def test_route_ties_live(torch_gpu, E):
    """Tie-heavy rows of every network size (maxN 8..256), top-k from 1 to 16,
    softmax with and without renormalisation, and sigmoid + bias with group
    limits: selection, order and weights bit-exact with the oracle's restated
    np.argpartition."""
    from fastllm_py.expert_router import route_topk_device

    rng = np.random.default_rng(880 + E)
    for k in [k for k in (1, 2, 4, 8, 16) if k <= E]:
        for scoring, norm in (("softmax", False), ("softmax", True), ("sigmoid", True)):
            levels = int(rng.integers(2, 9))
            vals = rng.standard_normal(levels).astype(np.float16)
            logits = vals[rng.integers(0, levels, size=(48, E))].astype(np.float32)
            kw = dict(norm_topk_prob=norm, scoring=scoring, routed_scaling=1.5)
            if scoring == "sigmoid":
                kw["e_score_bias"] = (vals[rng.integers(0, levels, size=E)] * 0.1).astype(np.float32)
                if E % 8 == 0 and E // 8 * 4 >= k:
                    kw.update(n_group=8, topk_group=4)
            r = route_topk_device(logits, k, **kw)
            _, ia, wa = R.route_topk(logits, k, return_arrays=True, **kw)
            ctx = f"E={E} k={k} {scoring} norm={norm}"
            np.testing.assert_array_equal(r["topk_ids"].cpu().numpy(), ia, err_msg=ctx)
            np.testing.assert_array_equal(r["topk_w"].cpu().numpy().view(np.uint32),
                                          wa.view(np.uint32), err_msg=ctx)


@pytest.mark.parametrize("T", [1, 16])
def test_moe_route_forward_ties(torch_gpu, T):
    """Tied logits through the one-call path (T = 1 routes inside the gate/up
    launch): routing outputs bit-exact with the restated np.argpartition."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    E, K, hidden, inter = 60, 4, 256, 256
    rng = np.random.default_rng(31 + T)
    st, _ = _stacked(_experts(rng, E, hidden, inter, 0.05), 128)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    for trial in range(6):
        vals = rng.standard_normal(3).astype(np.float16)
        logits = vals[rng.integers(0, 3, size=(T, E))].astype(np.float32)
        r = {}
        moe_int4.moe_route_forward(x, torch.from_numpy(logits).cuda(), st, K, E, hidden, inter,
                                   route=r)
        _, ia, wa = R.route_topk(logits, K, return_arrays=True)
        np.testing.assert_array_equal(r["topk_ids"].cpu().numpy(), ia, err_msg=str(trial))
        np.testing.assert_array_equal(r["topk_w"].cpu().numpy().view(np.uint32), wa.view(np.uint32))


def _check_lists(r, ids, w, T, K):
    """MoE lists vs the (T, K) selection: experts ascending, tokens ascending
    within an expert, every (token, expert, weight) listed once."""
    na = int(r["n_active"].cpu()[0])
    act = r["active"].cpu().numpy()[:na]
    offs = r["offsets"].cpu().numpy()[:na + 1]
    tok = r["tok"].cpu().numpy()
    tokw = r["tokw"].cpu().numpy()
    assert act.tolist() == sorted(set(ids.reshape(-1).tolist()))
    assert offs[0] == 0 and offs[-1] == T * K
    got = {}
    for s, e in enumerate(act.tolist()):
        ts = tok[offs[s]:offs[s + 1]]
        assert np.all(np.diff(ts) > 0)
        for p in range(offs[s], offs[s + 1]):
            got[(int(tok[p]), e)] = np.float32(tokw[p])
    want = {(t, int(ids[t, i])): np.float32(w[t, i]) for t in range(T) for i in range(K)}
    assert got == want


@pytest.mark.parametrize("T,E,k", [(1, 60, 4), (16, 60, 4), (5, 256, 8), (16, 128, 16),
                                   (40, 128, 8), (512, 128, 8)])
def test_route_lists(torch_gpu, T, E, k):
    """Router-built MoE lists (one-workgroup path T <= 16, separate list kernel
    above) agree with the router's own (T, k) selection."""
    from fastllm_py.expert_router import route_topk_device

    rng = np.random.default_rng(T * 1000 + E)
    s = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    r = route_topk_device(s, k)
    _check_lists(r, r["topk_ids"].cpu().numpy(), r["topk_w"].cpu().numpy(), T, k)


def test_build_lists_slot_and_dense(torch_gpu):
    """Explicit slot lists: slot order kept, zero weights and out-of-range
    experts dropped."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    T, E = 3, 10
    cand = torch.tensor([7, 2, 7, 11, 4], dtype=torch.int32, device="cuda")
    coef = torch.tensor([[0.5, 0.0, 1.0], [0.0, 0.0, 0.0], [2.0, 3.0, 0.0],
                         [1.0, 1.0, 1.0], [0.0, 4.0, 0.25]], device="cuda")
    L = moe_int4.build_lists(T, E, slot_coef=coef, cand=cand)
    na = int(L["n_active"].cpu()[0])
    assert na == 3
    assert L["active"].cpu().tolist()[:3] == [7, 7, 4]
    assert L["offsets"].cpu().tolist()[:4] == [0, 2, 4, 6]
    assert L["tok"].cpu().tolist()[:6] == [0, 2, 0, 1, 1, 2]
    assert L["tokw"].cpu().tolist()[:6] == [0.5, 1.0, 2.0, 3.0, 4.0, 0.25]
    rw = torch.zeros((T, E), device="cuda")
    rw[0, 3], rw[2, 3], rw[1, 9] = 1.5, 0.5, 2.0
    D = moe_int4.build_lists(T, E, rw=rw)
    assert int(D["n_active"].cpu()[0]) == 2
    assert D["active"].cpu().tolist()[:2] == [3, 9]
    assert D["tok"].cpu().tolist()[:3] == [0, 2, 1]


# ---------------------------------------------------------------- fused MoE
@pytest.mark.parametrize("E,K,hidden,inter,gs", [(8, 4, 256, 512, 128), (60, 4, 512, 1408, 128),
                                                 (4, 1, 128, 256, 32)])
def test_fused_moe_matches_reference(torch_gpu, E, K, hidden, inter, gs):
    # reference tests/test_moe_int4.py:23-54
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(2)
    experts = _experts(rng, E, hidden, inter)
    x = (rng.standard_normal(hidden) * 0.5).astype(np.float32)
    eidx = rng.choice(E, size=K, replace=False).astype(np.int32)
    rw = (rng.random(K) + 0.1).astype(np.float32)
    stacked, stacked_o = _stacked(experts, gs)
    xd = torch.from_numpy(x).cuda()
    y = moe_int4.fused_moe_ffn(xd, stacked, torch.from_numpy(eidx).cuda(),
                               torch.from_numpy(rw).cuda(), hidden, inter).cpu().numpy()
    y2 = moe_int4.fused_moe_ffn2(xd, stacked, torch.from_numpy(eidx).cuda(),
                                 torch.from_numpy(rw).cuda(), hidden, inter).cpu().numpy()
    deq = OM.dequant_stacked(stacked_o, gs)
    ref = OM.moe_ref(x[None], deq, eidx[None], rw[None])[0]
    assert Q.max_abs_rel(y, ref) < 5e-3
    assert Q.max_abs_rel(y2, y) < 1e-6  # same kernels; fp32 atomics may reorder the sum


def test_fused_moe_weighted_matches_index_version(torch_gpu):
    # reference tests/test_moe_int4.py:67-85
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(4)
    E, K, hidden, inter, gs = 60, 4, 512, 1408, 128
    stacked, stacked_o = _stacked(_experts(rng, E, hidden, inter), gs)
    x = torch.from_numpy((rng.standard_normal(hidden) * 0.3).astype(np.float32)).cuda()
    eidx = np.sort(rng.choice(E, K, replace=False)).astype(np.int32)
    w = (rng.random(K) + 0.1).astype(np.float32)
    rw = np.zeros(E, dtype=np.float32)
    rw[eidx] = w
    yw = moe_int4.fused_moe_weighted(x, stacked, torch.from_numpy(rw).cuda(), E, hidden, inter,
                                     aidx=torch.from_numpy(eidx).cuda())
    yi = moe_int4.fused_moe_ffn2(x, stacked, torch.from_numpy(eidx).cuda(),
                                 torch.from_numpy(w).cuda(), hidden, inter)
    assert Q.max_abs_rel(yw.cpu().numpy(), yi.cpu().numpy()) < 1e-6
    # no aidx: every expert visited, zero weights contribute nothing
    yall = moe_int4.fused_moe_weighted(x, stacked, torch.from_numpy(rw).cuda(), E, hidden, inter)
    np.testing.assert_allclose(yall.cpu().numpy(), yw.cpu().numpy(), rtol=1e-5, atol=1e-6)


def _qwen15_layer(torch, rng, E=60, hidden=2048, inter=1408, sinter=5632):
    from fastllm_py.kernels import moe_int4

    experts = _experts(rng, E, hidden, inter, 0.02)
    shared = _experts(rng, 1, hidden, sinter, 0.02)
    st, st_o = _stacked(experts, 128)
    sh, sh_o = _stacked(shared, 128)
    sgw = (rng.standard_normal((1, hidden)) * 0.02).astype(np.float16)
    gw = (rng.standard_normal((E, hidden)) * 0.02).astype(np.float16)
    return st, sh, sgw, gw, st_o, sh_o


@pytest.mark.parametrize("T", [1, 16])
def test_moe_layer_config4(torch_gpu, T):
    """BASELINE config 4 (Qwen1.5-MoE-A2.7B): fp16 router logits ~ N(0,1),
    top-4 softmax, shared expert 5632 with sigmoid gate.  Routing bit-exact vs
    the golden fixture; output vs the fp32 oracle."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    g = np.load(os.path.join(GOLDEN, f"route_qwen15moe_t{T}.npz"))
    rng = np.random.default_rng(4100 + T)
    st, sh, sgw, _, st_o, sh_o = _qwen15_layer(torch, rng)
    hidden, inter, sinter, E = 2048, 1408, 5632, 60
    x = rng.standard_normal((T, hidden)).astype(np.float16).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    sl = xd @ torch.from_numpy(sgw.astype(np.float32)).cuda().T
    r = route_topk_device(g["logits"], 4, shared_logit=sl.reshape(-1))
    np.testing.assert_array_equal(r["topk_ids"].cpu().numpy(), g["idx_argpartition"])
    np.testing.assert_array_equal(r["topk_w"].cpu().numpy().view(np.uint32),
                                  g["w_argpartition"].view(np.uint32))
    y = moe_int4.moe_forward(xd, st, E, hidden, inter, r, max_slots=min(E, 4 * T),
                             max_entries=4 * T, shared=sh, shared_inter=sinter,
                             shared_coef=r["shared_coef"])
    coef = 1.0 / (1.0 + np.exp(-sl.reshape(-1).cpu().numpy()))
    ref = OM.moe_ref(x, OM.dequant_stacked(st_o, 128), g["idx_argpartition"],
                     g["w_argpartition"], OM.dequant_stacked(sh_o, 128), coef)
    assert Q.max_abs_rel(y.cpu().numpy(), ref) < 1e-2
    assert Q.max_abs_rel(y.cpu().numpy(), ref) < 5e-3


def test_moe_branch_graph_capture(torch_gpu):
    """gate matvec + router + fused MoE captured in one HIP graph: every replay
    (with eager work in between) equals the eager result up to the fp32
    atomic summation order of the down projection."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(5)
    E, K, hidden, inter, sinter = 60, 4, 512, 512, 1024
    st, st_o = _stacked(_experts(rng, E, hidden, inter), 128)
    sh, sh_o = _stacked(_experts(rng, 1, hidden, sinter), 128)
    gw = torch.from_numpy((rng.standard_normal((E, hidden)) * 0.1).astype(np.float16)).cuda()
    sgw = torch.from_numpy((rng.standard_normal((1, hidden)) * 0.1).astype(np.float16)).cuda()
    x = torch.from_numpy((rng.standard_normal((1, hidden)) * 0.5).astype(np.float32)).cuda()
    eager = moe_int4.moe_branch(x, gw, st, K, E=E, hidden=hidden, inter=inter, shared=sh,
                                shared_inter=sinter, shared_gate_w=sgw).clone()
    bufs = {"logits": torch.empty((1, E), device="cuda"), "slogit": torch.empty(1, device="cuda"),
            "out": torch.empty((1, hidden), device="cuda")}
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for _ in range(2):
            moe_int4.moe_branch(x, gw, st, K, E=E, hidden=hidden, inter=inter, shared=sh,
                                shared_inter=sinter, shared_gate_w=sgw, bufs=bufs)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = moe_int4.moe_branch(x, gw, st, K, E=E, hidden=hidden, inter=inter, shared=sh,
                                  shared_inter=sinter, shared_gate_w=sgw, bufs=bufs)
    for i in range(4):
        bufs["out"].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert Q.max_abs_rel(out.cpu().numpy(), eager.cpu().numpy()) < 1e-6, i
        _ = (x * 2).sum().item()  # eager work between replays


@pytest.mark.parametrize("T,E,K,hidden,inter,sinter,gs", [
    (3, 16, 4, 512, 768, 1536, 128),      # 6 down blocks, shared in 2 pieces
    (16, 8, 2, 256, 256, 0, 64),          # no shared expert, group 64
    (2, 4, 2, 4096, 640, 2560, 128),      # hidden 4096: 4 gate/up blocks per wave
    (1, 2, 1, 1024, 8192, 0, 128),        # inter 8192: 8 down blocks per wave
    (5, 6, 3, 384, 384, 3200, 32),        # group 32, shared in 9 pieces
    # 5..16 tokens, hidden a multiple of 256: the column-split down kernel
    (8, 12, 4, 512, 2048, 2560, 128),     # 16 k blocks (8 chunks), shared in 2 pieces
    (7, 10, 3, 768, 640, 1152, 64),       # 5 k blocks (a chunk half past the end), shared 6 + 3
])
def test_fused_moe_shapes(torch_gpu, T, E, K, hidden, inter, sinter, gs):
    """Router lists + fused MoE over the launch-plan variants, vs the fp32
    oracle; a second identical call agrees up to the atomic summation order."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(T * 7 + hidden)
    st, st_o = _stacked(_experts(rng, E, hidden, inter, 0.05), gs)
    sh, sh_o = _stacked(_experts(rng, 1, hidden, sinter, 0.05), gs) if sinter else (None, None)
    x = (rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    sl = rng.standard_normal(T).astype(np.float32)
    r = route_topk_device(logits, K, norm_topk_prob=True,
                          shared_logit=sl if sinter else None)
    xd = torch.from_numpy(x).cuda()
    kw = dict(max_slots=min(E, T * K), max_entries=T * K, shared=sh, shared_inter=sinter,
              shared_coef=r.get("shared_coef"))
    y = moe_int4.moe_forward(xd, st, E, hidden, inter, r, **kw)
    y2 = moe_int4.moe_forward(xd, st, E, hidden, inter, r, **kw)
    assert Q.max_abs_rel(y2.cpu().numpy(), y.cpu().numpy()) < 1e-6
    ids, w = r["topk_ids"].cpu().numpy(), r["topk_w"].cpu().numpy()
    coef = 1.0 / (1.0 + np.exp(-sl)) if sinter else None
    ref = OM.moe_ref(x, OM.dequant_stacked(st_o, gs), ids, w,
                     OM.dequant_stacked(sh_o, gs) if sh else None, coef)
    assert Q.max_abs_rel(y.cpu().numpy(), ref) < 5e-3


@pytest.mark.parametrize("T,E,K,hidden,inter,sinter,gs,norm", [
    (1, 60, 4, 2048, 1408, 5632, 128, False),  # config 4, one token
    (16, 60, 4, 2048, 1408, 5632, 128, False),  # config 4, 16 tokens
    (3, 16, 4, 512, 768, 1536, 128, True),
    (16, 128, 16, 256, 256, 0, 64, True),        # 256 entries, group 64
    (5, 6, 3, 384, 384, 3200, 32, False),         # group 32, shared in 9 pieces
    # one token: routed inside the gate/up launch (the Qwen3-30B-A3B decode
    # shape: eight slots, down with one block per wave)
    (1, 128, 8, 2048, 768, 0, 128, True),
    (1, 16, 4, 512, 768, 1536, 128, True),
    (1, 128, 16, 256, 256, 0, 64, True),
    (1, 6, 3, 384, 384, 3200, 32, False),
])
def test_moe_route_forward(torch_gpu, T, E, K, hidden, inter, sinter, gs, norm):
    """Router + fused MoE in one native call: routing outputs bit-exact vs the
    router entry, y vs the two-call path (up to the atomic summation order)
    and vs the fp32 oracle, over three calls in a row and a second stream."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(9000 + T * 13 + E + hidden)
    st, st_o = _stacked(_experts(rng, E, hidden, inter, 0.05), gs)
    sh, sh_o = _stacked(_experts(rng, 1, hidden, sinter, 0.05), gs) if sinter else (None, None)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda() if sinter else None
    ref_r = route_topk_device(logits, K, norm_topk_prob=norm, shared_logit=sl)
    y2 = moe_int4.moe_forward(x, st, E, hidden, inter, ref_r, max_slots=min(E, T * K),
                              max_entries=T * K, shared=sh, shared_inter=sinter,
                              shared_coef=ref_r.get("shared_coef"))
    ids, w = ref_r["topk_ids"].cpu().numpy(), ref_r["topk_w"].cpu().numpy()
    coef = 1.0 / (1.0 + np.exp(-sl.cpu().numpy())) if sinter else None
    ref = OM.moe_ref(x.cpu().numpy(), OM.dequant_stacked(st_o, gs), ids, w,
                     OM.dequant_stacked(sh_o, gs) if sh else None, coef)
    s2 = torch.cuda.Stream()
    for call in range(4):
        stream = s2 if call == 3 else None
        r = {}
        with torch.cuda.stream(s2 if stream is not None else torch.cuda.current_stream()):
            y = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, norm_topk_prob=norm,
                                           shared=sh, shared_inter=sinter, shared_logit=sl,
                                           route=r, stream=stream)
        torch.cuda.synchronize()
        for k in ("topk_ids", "topk_w", "rw", "n_active"):
            np.testing.assert_array_equal(r[k].cpu().numpy().view(np.uint32),
                                          ref_r[k].cpu().numpy().view(np.uint32), err_msg=k)
        na = int(r["n_active"].item())
        n_ent = int(ref_r["offsets"][na].item())
        for k, n in (("active", na), ("offsets", na + 1), ("tok", n_ent), ("tokw", n_ent)):
            np.testing.assert_array_equal(r[k][:n].cpu().numpy().view(np.uint32),
                                          ref_r[k][:n].cpu().numpy().view(np.uint32), err_msg=k)
        if sinter:
            np.testing.assert_array_equal(r["shared_coef"].cpu().numpy().view(np.uint32),
                                          ref_r["shared_coef"].cpu().numpy().view(np.uint32))
        yc = y.cpu().numpy()
        assert np.isfinite(yc).all(), call
        assert Q.max_abs_rel(yc, y2.cpu().numpy()) < 1e-5, call
        assert Q.max_abs_rel(yc, ref) < 5e-3, call


@pytest.mark.parametrize("T", [1, 4, 12, 40, 130])
def test_moe_route_forward_sigmoid_groups(torch_gpu, T):
    """Sigmoid scoring with a score bias, group-limited selection and routed
    scaling through the one-call path (T = 1 routes inside the gate/up
    launch; above 16 tokens the router's last workgroup builds the lists):
    routing bit-exact vs the router entry, y vs the two-call path."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(9100 + T)
    E, K, hidden, inter, sinter, gs = 64, 6, 512, 256, 768, 128
    kw = dict(norm_topk_prob=True, scoring="sigmoid", routed_scaling=2.5,
              e_score_bias=torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).cuda(),
              n_group=8, topk_group=3)
    st, st_o = _stacked(_experts(rng, E, hidden, inter, 0.05), gs)
    sh, sh_o = _stacked(_experts(rng, 1, hidden, sinter, 0.05), gs)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda()
    ref_r = route_topk_device(logits, K, shared_logit=sl, **kw)
    y2 = moe_int4.moe_forward(x, st, E, hidden, inter, ref_r, max_slots=min(E, T * K),
                              max_entries=T * K, shared=sh, shared_inter=sinter,
                              shared_coef=ref_r["shared_coef"])
    for _ in range(2):
        r = {}
        y = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, shared=sh,
                                       shared_inter=sinter, shared_logit=sl, route=r, **kw)
        torch.cuda.synchronize()
        for k in ("topk_ids", "topk_w", "rw", "n_active", "shared_coef"):
            np.testing.assert_array_equal(r[k].cpu().numpy().view(np.uint32),
                                          ref_r[k].cpu().numpy().view(np.uint32), err_msg=k)
        na = int(r["n_active"].item())
        n_ent = int(ref_r["offsets"][na].item())
        for k, n in (("active", na), ("offsets", na + 1), ("tok", n_ent), ("tokw", n_ent)):
            np.testing.assert_array_equal(r[k][:n].cpu().numpy().view(np.uint32),
                                          ref_r[k][:n].cpu().numpy().view(np.uint32), err_msg=k)
        assert Q.max_abs_rel(y.cpu().numpy(), y2.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("hidden,inter,gs", [(512, 384, 128), (256, 640, 32)])
def test_stack_marlin_experts_bit_exact(torch_gpu, hidden, inter, gs):
    """Resident Marlin payloads -> stacked tile layout on the GPU: the tiles are
    the oracle's tile pack of the very integers, scales and zeros the Marlin
    quantizer produced, and the fused MoE over them matches the oracle on the
    Marlin-dequantized weights."""
    from fastllm_py.kernels import moe_int4
    from fastllm_py.moe import quantize_marlin_matrix_device

    torch = torch_gpu
    rng = np.random.default_rng(6100 + hidden + gs)
    E, K = 3, 2
    exps = _experts(rng, E, hidden, inter, 0.05)
    pays = [{p: quantize_marlin_matrix_device(torch.from_numpy(w[p].astype(np.float32)).cuda(), gs)
             for p in ("gate", "up", "down")} for w in exps]
    st = moe_int4.stack_marlin_experts(pays, gs)
    deq = {}
    for proj in ("gate", "up", "down"):
        ws = [w[proj].astype(np.float32) for w in exps]
        qs, hats = [], []
        for W in ws:
            q, s, z = Q.quantize_int4_marlin(W, gs)
            s16, zp = Q.marlin_scales_zeros(s, z)
            hats.append(Q.marlin_dequant(q, s16, zp, gs))
            qs.append(Q.moe_tile_pack(Q._pack_pairs(q), s.astype(np.float16), z.astype(np.float16)))
        np.testing.assert_array_equal(st[f"{proj}.qtile"].cpu().numpy(),
                                      np.stack([a for a, _ in qs]).reshape(st[f"{proj}.qtile"].shape))
        np.testing.assert_array_equal(st[f"{proj}.sz"].cpu().numpy().view(np.uint32),
                                      np.stack([b for _, b in qs]).reshape(st[f"{proj}.sz"].shape))
        deq[proj] = np.stack(hats)
    from fastllm_py.expert_router import route_topk_device

    T = 2
    x = (rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
    r = route_topk_device(logits, K)
    y = moe_int4.moe_forward(torch.from_numpy(x).cuda(), st, E, hidden, inter, r, max_slots=E,
                             max_entries=T * K)
    ref = OM.moe_ref(x, deq, r["topk_ids"].cpu().numpy(), r["topk_w"].cpu().numpy())
    assert Q.max_abs_rel(y.cpu().numpy(), ref) < 5e-3


def test_fused_moe_edge_lists(torch_gpu):
    """ffn2 with a repeated expert (two slots, summed), zero weights (dropped)
    and all-zero routing without a shared expert (y == 0)."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(12)
    E, hidden, inter = 6, 256, 384
    st, st_o = _stacked(_experts(rng, E, hidden, inter), 128)
    deq = OM.dequant_stacked(st_o, 128)
    x = (rng.standard_normal(hidden) * 0.5).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    eidx = np.array([3, 1, 3, 5], np.int32)
    rw = np.array([0.5, 0.0, 0.25, 1.0], np.float32)
    y = moe_int4.fused_moe_ffn2(xd, st, torch.from_numpy(eidx).cuda(),
                                torch.from_numpy(rw).cuda(), hidden, inter).cpu().numpy()
    ref = OM.moe_ref(x[None], deq, eidx[None], rw[None])[0]
    assert Q.max_abs_rel(y, ref) < 5e-3
    z = moe_int4.fused_moe_weighted(xd, st, torch.zeros(E, device="cuda"), E, hidden, inter)
    assert torch.count_nonzero(z).item() == 0


@pytest.mark.parametrize("T,E,K,hidden,inter,sinter,gs,norm", [
    (17, 8, 2, 256, 256, 0, 128, True),     # just past the decode kernels
    (64, 16, 4, 512, 384, 1024, 64, False),  # shared expert, group 64
    (100, 32, 8, 512, 768, 0, 32, True),     # ragged 64-row chunks, group 32
    (300, 4, 4, 256, 128, 256, 128, False),  # every expert holds all 300 tokens
])
def test_fused_moe_prefill(torch_gpu, T, E, K, hidden, inter, sinter, gs, norm):
    """T > 16: router lists + the grouped-GEMM MoE kernels vs the fp32 oracle
    (expert-grouped evaluation, pinned to the per-token oracle on the CPU);
    a second call agrees up to the atomic summation order."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(T * 13 + hidden + E)
    st, st_o = _stacked(_experts(rng, E, hidden, inter, 0.05), gs)
    sh, sh_o = _stacked(_experts(rng, 1, hidden, sinter, 0.05), gs) if sinter else (None, None)
    x = (rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)
    sl = rng.standard_normal(T).astype(np.float32)
    r = route_topk_device(logits, K, norm_topk_prob=norm, shared_logit=sl if sinter else None)
    xd = torch.from_numpy(x).cuda()
    kw = dict(max_slots=min(E, T * K), max_entries=T * K, shared=sh, shared_inter=sinter,
              shared_coef=r.get("shared_coef"))
    y = moe_int4.moe_forward(xd, st, E, hidden, inter, r, **kw)
    # repeats agree up to the atomic order (the activation ring of the
    # grouped INT4 GEMM once let a past-end copy overwrite the last block's
    # stage under slower waves; run-to-run differences showed it)
    for _ in range(4):
        y2 = moe_int4.moe_forward(xd, st, E, hidden, inter, r, **kw)
        assert Q.max_abs_rel(y2.cpu().numpy(), y.cpu().numpy()) < 1e-6
    ids, w = r["topk_ids"].cpu().numpy(), r["topk_w"].cpu().numpy()
    coef = 1.0 / (1.0 + np.exp(-sl)) if sinter else None
    ref = OM.moe_ref_grouped(x, OM.dequant_stacked(st_o, gs), ids, w,
                             OM.dequant_stacked(sh_o, gs) if sh else None, coef)
    assert Q.max_abs_rel(y.cpu().numpy(), ref) < 5e-3


def test_moe_prefill_config5(torch_gpu):
    """BASELINE config 5 (Qwen3-30B-A3B MoE layer at M=512): 128 experts,
    hidden 2048, inter 768, top-8 softmax with renormalisation from fp16
    logits ~ N(0,1); routing bit-exact vs the golden fixture, output vs the
    fp32 oracle."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    g = np.load(os.path.join(GOLDEN, "route_qwen3moe_t512.npz"))
    T, E, K, hidden, inter = 512, 128, 8, 2048, 768
    rng = np.random.default_rng(5512)
    experts = _experts(rng, E, hidden, inter, 0.02)
    st, st_o = _stacked(experts, 128)
    del experts
    x = rng.standard_normal((T, hidden)).astype(np.float16).astype(np.float32)
    r = route_topk_device(g["logits"], K, norm_topk_prob=True)
    ids = r["topk_ids"].cpu().numpy()
    w = r["topk_w"].cpu().numpy()
    np.testing.assert_array_equal(ids, g["idx_argpartition"])
    np.testing.assert_array_equal(w.view(np.uint32), g["w_argpartition"].view(np.uint32))
    y = moe_int4.moe_forward(torch.from_numpy(x).cuda(), st, E, hidden, inter, r,
                             max_slots=E, max_entries=T * K)
    ref = OM.moe_ref_grouped(x, OM.dequant_stacked(st_o, 128), ids, w)
    assert Q.max_abs_rel(y.cpu().numpy(), ref) < 5e-3
    # the one-call routed entry (router's last workgroup builds the lists):
    # the same routing and lists bit for bit, y up to the atomic order
    o = {}
    ws = torch.zeros(moe_int4.moe_workspace_bytes(T, hidden, inter, 0, T * K), dtype=torch.uint8,
                     device="cuda")
    for _ in range(2):  # the second call finds the arrival counter back at zero
        y2 = moe_int4.moe_route_forward(torch.from_numpy(x).cuda(), torch.from_numpy(g["logits"]).cuda(),
                                        st, K, E, hidden, inter, norm_topk_prob=True, route=o,
                                        workspace=ws)
        torch.cuda.synchronize()
        _assert_same_lists(o, r)
        assert Q.max_abs_rel(y2.cpu().numpy(), y.cpu().numpy()) < 1e-6


def test_routed_prefill_graph_replays(torch_gpu):
    """The routed entry above 16 tokens captured in a HIP graph: every replay
    (eager work and synchronisations between them) gives the eager call's
    lists bit for bit and its y up to the atomic order -- the router's
    arrival counter is back at zero after each replay."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    T, E, K, hidden, inter = 96, 16, 4, 512, 256
    rng = np.random.default_rng(9601)
    st, _ = _stacked(_experts(rng, E, hidden, inter, 0.05), 128)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    ws = torch.zeros(moe_int4.moe_workspace_bytes(T, hidden, inter, 0, T * K), dtype=torch.uint8,
                     device="cuda")
    eager_r = {}
    eager = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, route=eager_r, workspace=ws)
    torch.cuda.synchronize()
    r = moe_int4.alloc_route_buffers(T, E, K)
    out = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):  # warm-up outside capture (workspace and buffers exist)
        moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, route=r, out=out, workspace=ws,
                                   stream=s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, route=r, out=out, workspace=ws,
                                   stream=s)
    for _ in range(3):
        out.zero_()
        for k in ("tok", "tokw", "active", "offsets"):
            r[k].fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        _assert_same_lists(r, eager_r)
        assert Q.max_abs_rel(out.cpu().numpy(), eager.cpu().numpy()) < 1e-6


def _assert_same_lists(a, b):
    """Router outputs and MoE lists of two routings are identical."""
    for k in ("topk_ids", "topk_w", "n_active"):
        np.testing.assert_array_equal(a[k].cpu().numpy(), b[k].cpu().numpy(), err_msg=k)
    na = int(a["n_active"].item())
    np.testing.assert_array_equal(a["active"].cpu().numpy()[:na], b["active"].cpu().numpy()[:na])
    off = a["offsets"].cpu().numpy()[:na + 1]
    np.testing.assert_array_equal(off, b["offsets"].cpu().numpy()[:na + 1])
    n = int(off[-1])
    np.testing.assert_array_equal(a["tok"].cpu().numpy()[:n], b["tok"].cpu().numpy()[:n])
    np.testing.assert_array_equal(a["tokw"].cpu().numpy()[:n], b["tokw"].cpu().numpy()[:n])


@pytest.mark.parametrize("T,E,K,hidden,inter,sinter,gs,norm", [
    (17, 8, 2, 256, 256, 0, 128, True),      # five routing workgroups, the last holds one token
    (64, 16, 4, 512, 384, 1024, 64, False),  # shared expert with its sigmoid gate, group 64
    (300, 60, 4, 512, 256, 512, 128, False),  # E = 60 (one expert per lane)
    (200, 256, 8, 256, 256, 0, 128, True),   # E = 256, ragged 32-token bitmap words
])
def test_routed_prefill(torch_gpu, T, E, K, hidden, inter, sinter, gs, norm):
    """moe_route_forward above 16 tokens (one native call: router whose last
    workgroup builds the lists while spare workgroups write the fp16 copy of
    x, then the grouped GEMMs) against route_topk_device + moe_forward: the
    same router outputs and lists bit for bit, y up to the atomic order, on
    three calls through one workspace (the arrival counter is left at zero);
    the deterministic combine bit-identical on a repeat; the no-alloc entry
    equal to the allocating one."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(T * 7 + E + hidden)
    st, st_o = _stacked(_experts(rng, E, hidden, inter, 0.05), gs)
    sh, _ = _stacked(_experts(rng, 1, hidden, sinter, 0.05), gs) if sinter else (None, None)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda() if sinter else None
    r = route_topk_device(logits, K, norm_topk_prob=norm, shared_logit=sl)
    kw = dict(shared=sh, shared_inter=sinter)
    y_ref = moe_int4.moe_forward(x, st, E, hidden, inter, r, max_slots=min(E, T * K),
                                 max_entries=T * K, shared_coef=r.get("shared_coef"), **kw)
    ws = torch.zeros(moe_int4.moe_workspace_bytes(T, hidden, inter, sinter, T * K), dtype=torch.uint8,
                     device="cuda")
    o = {}
    for _ in range(3):
        y = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, norm_topk_prob=norm,
                                       shared_logit=sl, route=o, workspace=ws, **kw)
        torch.cuda.synchronize()
        _assert_same_lists(o, r)
        if sinter:
            np.testing.assert_array_equal(o["shared_coef"].cpu().numpy(), r["shared_coef"].cpu().numpy())
        assert Q.max_abs_rel(y.cpu().numpy(), y_ref.cpu().numpy()) < 1e-6
    od = {}
    yd = [moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, norm_topk_prob=norm,
                                     shared_logit=sl, route=od, deterministic=True, **kw)
          for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(yd[0], yd[1])
    assert Q.max_abs_rel(yd[0].cpu().numpy(), y_ref.cpu().numpy()) < 1e-5
    bufs = moe_int4.alloc_route_buffers(T, E, K)
    out = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
    moe_int4.moe_route_forward_noalloc(x, logits, st, K, E, hidden, inter, route=bufs, out=out,
                                       norm_topk_prob=norm, shared_logit=sl, **kw)
    torch.cuda.synchronize()
    _assert_same_lists(bufs, r)
    assert Q.max_abs_rel(out.cpu().numpy(), y_ref.cpu().numpy()) < 1e-6

"""The fused MoE's deterministic combine (fastllm_moe_fused_ex /
fastllm_moe_routed_ex with FASTLLM_MOE_DETERMINISTIC) on the GPU.

Without the flag the down projections add their terms into y with fp32
atomics (as the reference's moew_down, fastllm_py/kernels/moe_int4.py:250),
so the last bits of y depend on arrival order.  With it the terms go to the
workspace and one launch sums each token's terms in a fixed order.  Checked
here: repeated calls (and graph replays) give bit-identical y, for the decode
kernels (1..16 tokens, INT4 / FP8 / MXFP4 experts, shared expert split in
pieces) and the grouped prefill kernels; y agrees with the atomic path to
1e-5 and with the fp32 oracle to the same bound as the atomic path's tests.
"""
import numpy as np
import pytest

from oracle import moe as OM
from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _experts(rng, E, hidden, inter, scale=0.05):
    return [{"gate": (rng.standard_normal((inter, hidden)) * scale).astype(np.float16),
             "up": (rng.standard_normal((inter, hidden)) * scale).astype(np.float16),
             "down": (rng.standard_normal((hidden, inter)) * scale).astype(np.float16)}
            for _ in range(E)]


def _stacked(experts, gs):
    from fastllm_py.kernels import moe_int4

    st = moe_int4.build_stacked_experts(experts, gs)
    orc = {}
    for proj in ("gate", "up", "down"):
        p, s_, z = Q.quantize_int4_rowmajor(np.stack([e[proj] for e in experts]), gs)
        orc.update({f"{proj}.qweight": p, f"{proj}.scales": s_, f"{proj}.zeros": z})
    return st, orc


def _bits(y):
    return y.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("T,E,K,hidden,inter,sinter,gs,norm", [
    (1, 60, 4, 2048, 1408, 5632, 128, False),   # config 4, one token (routed in the gate/up launch)
    (16, 60, 4, 2048, 1408, 5632, 128, False),  # config 4, 16 tokens
    (5, 6, 3, 384, 384, 3200, 32, False),        # group 32, shared expert in 9 pieces
    (16, 128, 16, 256, 256, 0, 64, True),        # 256 entries, no shared expert
    (1, 128, 8, 2048, 768, 0, 128, True),        # Qwen3-30B-A3B decode shape
])
def test_det_decode_repeats_bit_identical(torch_gpu, T, E, K, hidden, inter, sinter, gs, norm):
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(7000 + T * 7 + E + hidden)
    st, st_o = _stacked(_experts(rng, E, hidden, inter), gs)
    sh, sh_o = _stacked(_experts(rng, 1, hidden, sinter), gs) if sinter else (None, None)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda() if sinter else None
    kw = dict(norm_topk_prob=norm, shared=sh, shared_inter=sinter, shared_logit=sl)
    r0 = {}
    y_atomic = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, route=r0, **kw)
    first = None
    for call in range(3):
        print(f"det decode T={T} E={E} call {call}", flush=True)
        r = {}
        y = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, route=r,
                                       deterministic=True, **kw)
        torch.cuda.synchronize()
        if first is None:
            first = _bits(y)
            ids, w = r["topk_ids"].cpu().numpy(), r["topk_w"].cpu().numpy()
            np.testing.assert_array_equal(ids, r0["topk_ids"].cpu().numpy())
            coef = 1.0 / (1.0 + np.exp(-sl.cpu().numpy())) if sinter else None
            ref = OM.moe_ref(x.cpu().numpy(), OM.dequant_stacked(st_o, gs), ids, w,
                             OM.dequant_stacked(sh_o, gs) if sh else None, coef)
            yc = y.cpu().numpy()
            assert np.isfinite(yc).all()
            assert Q.max_abs_rel(yc, y_atomic.cpu().numpy()) < 1e-5
            assert Q.max_abs_rel(yc, ref) < 5e-3
        else:
            np.testing.assert_array_equal(_bits(y), first, err_msg=f"call {call}")


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
@pytest.mark.parametrize("T", [1, 16])
def test_det_lowp_repeats_bit_identical(torch_gpu, fmt, T):
    """FP8 / MXFP4 experts: the same term rows and combine."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    E, K, hidden, inter, sinter = 16, 4, 1024, 512, 1536
    rng = np.random.default_rng(7100 + T + (0 if fmt == "fp8" else 50))

    def stack(n, o, i):
        w = (rng.standard_normal((n, o, i)) * 0.05).astype(np.float16).astype(np.float32)
        return w
    st = {"group": moe_int4.LOWP_FORMATS[fmt][1], "format": fmt}
    sh = dict(st)
    for d, n, inn in ((st, E, inter), (sh, 1, sinter)):
        for proj, (o, i) in (("gate", (inn, hidden)), ("up", (inn, hidden)), ("down", (hidden, inn))):
            d.update(moe_int4.stack_lowp(fmt, proj, stack(n, o, i)))
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda()
    kw = dict(shared=sh, shared_inter=sinter, shared_logit=sl)
    y_atomic = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, **kw)
    ys = [moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, deterministic=True, **kw)
          for _ in range(3)]
    torch.cuda.synchronize()
    assert Q.max_abs_rel(ys[0].cpu().numpy(), y_atomic.cpu().numpy()) < 1e-5
    for y in ys[1:]:
        np.testing.assert_array_equal(_bits(y), _bits(ys[0]))


@pytest.mark.parametrize("T,E,K,hidden,inter,sinter,gs,norm", [
    (64, 16, 4, 512, 384, 1024, 64, False),   # grouped kernels, shared expert
    (130, 32, 8, 512, 768, 0, 128, True),     # ragged 64-row chunks
])
def test_det_prefill_repeats_bit_identical(torch_gpu, T, E, K, hidden, inter, sinter, gs, norm):
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(7200 + T + E)
    st, st_o = _stacked(_experts(rng, E, hidden, inter), gs)
    sh, sh_o = _stacked(_experts(rng, 1, hidden, sinter), gs) if sinter else (None, None)
    x = (rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)
    sl = rng.standard_normal(T).astype(np.float32)
    r = route_topk_device(logits, K, norm_topk_prob=norm, shared_logit=sl if sinter else None)
    xd = torch.from_numpy(x).cuda()
    kw = dict(max_slots=min(E, T * K), max_entries=T * K, shared=sh, shared_inter=sinter,
              shared_coef=r.get("shared_coef"))
    y_atomic = moe_int4.moe_forward(xd, st, E, hidden, inter, r, **kw)
    ys = [moe_int4.moe_forward(xd, st, E, hidden, inter, r, deterministic=True, **kw)
          for _ in range(3)]
    torch.cuda.synchronize()
    ids, w = r["topk_ids"].cpu().numpy(), r["topk_w"].cpu().numpy()
    coef = 1.0 / (1.0 + np.exp(-sl)) if sinter else None
    ref = OM.moe_ref_grouped(x, OM.dequant_stacked(st_o, gs), ids, w,
                             OM.dequant_stacked(sh_o, gs) if sh else None, coef)
    assert Q.max_abs_rel(ys[0].cpu().numpy(), ref) < 5e-3
    assert Q.max_abs_rel(ys[0].cpu().numpy(), y_atomic.cpu().numpy()) < 1e-5
    for y in ys[1:]:
        np.testing.assert_array_equal(_bits(y), _bits(ys[0]))


def test_det_graph_replays_bit_identical(torch_gpu):
    """The deterministic call captured in a HIP graph: every replay (with
    eager work in between) equals the eager deterministic result bit for
    bit."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    T, E, K, hidden, inter, sinter = 16, 60, 4, 1024, 768, 1536
    rng = np.random.default_rng(7300)
    st, _ = _stacked(_experts(rng, E, hidden, inter), 128)
    sh, _ = _stacked(_experts(rng, 1, hidden, sinter), 128)
    x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
    sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda()
    route = moe_int4.alloc_route_buffers(T, E, K)
    ws = torch.empty((moe_int4.moe_workspace_bytes(T, hidden, inter, sinter, T * K, True),),
                     dtype=torch.uint8, device="cuda")
    y = torch.empty((T, hidden), dtype=torch.float32, device="cuda")

    def call(stream=None):
        return moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, shared=sh,
                                          shared_inter=sinter, shared_logit=sl, route=route,
                                          out=y, workspace=ws, stream=stream, deterministic=True)
    call()
    torch.cuda.synchronize()
    eager = _bits(y).copy()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call(torch.cuda.current_stream())
    for rep in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(y), eager, err_msg=f"replay {rep}")
        call()  # eager work between replays
        torch.cuda.synchronize()

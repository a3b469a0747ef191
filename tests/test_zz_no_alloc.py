"""fastllm_moe_int4_routed_noalloc (static-scratch router + fused MoE) against
fastllm_moe_int4_routed with a caller workspace, through the C ABI.

Two calls in a row on the same GPU scratch, the second with fewer tokens
(and so a smaller workspace need), each checked against the workspace entry:
routing outputs bit-exact, y within 1e-5 (the down projection adds with fp32
atomics, so only the summation order differs) and within 5e-3 of the fp32
oracle.  A shape whose workspace exceeds the 16 MiB scratch is refused before
anything is launched.
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


def _np_stacked(st):
    from fastllm_py.kernels import moe_int4

    return {k: (v.cpu().numpy() if hasattr(v, "cpu") else v)
            for k, v in moe_int4.unpack_stacked(st).items()}


def test_noalloc_matches_workspace_entry(torch_gpu):
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    E, K, hidden, inter, sinter, gs = 60, 4, 2048, 1408, 5632, 128  # Qwen1.5-MoE
    rng = np.random.default_rng(4242)
    st = moe_int4.build_stacked_experts(_experts(rng, E, hidden, inter), gs)
    sh = moe_int4.build_stacked_experts(_experts(rng, 1, hidden, sinter), gs)
    dq_st = OM.dequant_stacked(_np_stacked(st), gs)
    dq_sh = OM.dequant_stacked(_np_stacked(sh), gs)
    for call, T in enumerate((16, 1)):  # second call: fewer tokens
        x = torch.from_numpy((rng.standard_normal((T, hidden)) * 0.5).astype(np.float32)).cuda()
        logits = torch.from_numpy(
            rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)).cuda()
        sl = torch.from_numpy(rng.standard_normal(T).astype(np.float32)).cuda()
        r_ref = moe_int4.alloc_route_buffers(T, E, K)
        y_ref = moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, shared=sh,
                                           shared_inter=sinter, shared_logit=sl, route=r_ref)
        r = moe_int4.alloc_route_buffers(T, E, K)
        y = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
        print(f"noalloc call {call}: T={T}", flush=True)
        moe_int4.moe_route_forward_noalloc(x, logits, st, K, E, hidden, inter, route=r, out=y,
                                           shared=sh, shared_inter=sinter, shared_logit=sl)
        torch.cuda.synchronize()
        for k in ("topk_ids", "topk_w", "rw", "n_active", "shared_coef"):
            np.testing.assert_array_equal(r[k].cpu().numpy().view(np.uint32),
                                          r_ref[k].cpu().numpy().view(np.uint32), err_msg=k)
        na = int(r["n_active"].item())
        n_ent = int(r_ref["offsets"][na].item())
        for k, n in (("active", na), ("offsets", na + 1), ("tok", n_ent), ("tokw", n_ent)):
            np.testing.assert_array_equal(r[k][:n].cpu().numpy().view(np.uint32),
                                          r_ref[k][:n].cpu().numpy().view(np.uint32), err_msg=k)
        yc = y.cpu().numpy()
        assert np.isfinite(yc).all(), call
        assert Q.max_abs_rel(yc, y_ref.cpu().numpy()) < 1e-5, call
        coef = 1.0 / (1.0 + np.exp(-sl.cpu().numpy()))
        ref = OM.moe_ref(x.cpu().numpy(), dq_st, r["topk_ids"].cpu().numpy(),
                         r["topk_w"].cpu().numpy(), dq_sh, coef)
        assert Q.max_abs_rel(yc, ref) < 5e-3, call


def test_noalloc_refuses_oversized_workspace(torch_gpu):
    """T = 16, top-16 of 64 experts with a 32768-wide shared expert needs
    (256 + 16) x 32768 x 2 bytes of workspace, more than the 16 MiB scratch:
    refused (ValueError from rc 1) before any launch."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    T, E, K, hidden, inter, sinter = 16, 64, 16, 256, 256, 32768
    assert moe_int4.moe_workspace_bytes(T, hidden, inter, sinter, T * K) > 16 << 20
    rng = np.random.default_rng(1)
    st = moe_int4.build_stacked_experts(_experts(rng, E, hidden, inter), 128)
    sh = moe_int4.build_stacked_experts(_experts(rng, 1, hidden, sinter), 128)
    x = torch.zeros((T, hidden), dtype=torch.float32, device="cuda")
    logits = torch.zeros((T, E), dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    r = moe_int4.alloc_route_buffers(T, E, K)
    with pytest.raises(ValueError):
        moe_int4.moe_route_forward_noalloc(x, logits, st, K, E, hidden, inter, route=r, out=y,
                                           shared=sh, shared_inter=sinter)
    torch.cuda.synchronize()


def test_noalloc_refuses_wrongly_typed_vectors(torch_gpu):
    """shared_logit (T,) and e_score_bias (E,) reach the kernel as raw
    pointers: a host tensor, an fp16 tensor or a wrong length is a
    ValueError before any launch."""
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    T, E, K, hidden, inter, sinter = 2, 64, 4, 256, 256, 512
    rng = np.random.default_rng(2)
    st = moe_int4.build_stacked_experts(_experts(rng, E, hidden, inter), 128)
    sh = moe_int4.build_stacked_experts(_experts(rng, 1, hidden, sinter), 128)
    x = torch.zeros((T, hidden), dtype=torch.float32, device="cuda")
    logits = torch.zeros((T, E), dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    r = moe_int4.alloc_route_buffers(T, E, K)
    bad = {"shared_logit": (torch.zeros(T), torch.zeros(T, device="cuda").half(),
                            torch.zeros(T + 1, device="cuda")),
           "e_score_bias": (torch.zeros(E), torch.zeros(E, device="cuda").half(),
                            torch.zeros(E - 1, device="cuda"))}
    for name, vals in bad.items():
        for v in vals:
            kw = {name: v}
            if name == "e_score_bias":
                kw["scoring"] = "sigmoid"
            with pytest.raises(ValueError, match=name):
                moe_int4.moe_route_forward_noalloc(x, logits, st, K, E, hidden, inter, route=r,
                                                   out=y, shared=sh, shared_inter=sinter, **kw)
    torch.cuda.synchronize()

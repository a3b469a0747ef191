"""Write the committed golden fixtures of tests/golden/*.npz.

Inputs follow BASELINE.json's seeded recipes; expected outputs come from the
numpy oracle (oracle/), whose functions are pinned in tests/test_oracle_*.py.
Re-run only when the oracle changes:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import quant as Q  # noqa: E402
from oracle import router as R  # noqa: E402


def routing():
    cases = {
        # config 4: Qwen1.5-MoE router, fp16 logits ~ N(0,1), top-4 softmax, no renorm
        "qwen15moe_t16": dict(seed=4016, T=16, E=60, k=4, norm=False, scoring="softmax"),
        "qwen15moe_t1": dict(seed=4001, T=1, E=60, k=4, norm=False, scoring="softmax"),
        # config 5: Qwen3-30B-A3B router, M=512 tokens, top-8 softmax with renorm
        "qwen3moe_t512": dict(seed=5000, T=512, E=128, k=8, norm=True, scoring="softmax"),
        # DeepSeek-V3-like: sigmoid + bias, 8 groups keep 4, top-8, routed scaling 2.5
        "deepseek_t32": dict(seed=6000, T=32, E=64, k=8, norm=True, scoring="sigmoid",
                             n_group=8, topk_group=4, scale=2.5),
    }
    # tie-heavy rows: fp16 logits (and biases) from a few distinct values, so
    # many tokens hold experts tied at the k-th selection value
    ties = {
        "ties_e60_k4": dict(seed=7001, T=96, E=60, k=4, norm=False, scoring="softmax", levels=6),
        "ties_e128_k8": dict(seed=7002, T=96, E=128, k=8, norm=True, scoring="softmax", levels=8),
        "ties_e256_k16": dict(seed=7003, T=48, E=256, k=16, norm=True, scoring="softmax",
                              levels=12),
        "ties_groups": dict(seed=7004, T=64, E=64, k=8, norm=True, scoring="sigmoid", n_group=8,
                            topk_group=4, scale=2.5, levels=4),
    }
    cases.update(ties)
    for name, c in cases.items():
        rng = np.random.default_rng(c["seed"])
        if "levels" in c:
            vals = rng.standard_normal(c["levels"]).astype(np.float16)
            logits = vals[rng.integers(0, c["levels"], size=(c["T"], c["E"]))]
            bias = (vals[rng.integers(0, c["levels"], size=c["E"])].astype(np.float32) * 0.1
                    if c["scoring"] == "sigmoid" else None)
        else:
            logits = rng.standard_normal((c["T"], c["E"])).astype(np.float16)
            bias = (rng.standard_normal(c["E"]) * 0.1).astype(np.float32) if c["scoring"] == "sigmoid" else None
        kw = dict(norm_topk_prob=c["norm"], scoring=c["scoring"], routed_scaling=c.get("scale", 1.0),
                  e_score_bias=bias, n_group=c.get("n_group", 0), topk_group=c.get("topk_group", 0))
        s32 = logits.astype(np.float32)
        _, ia, wa = R.route_topk(s32, c["k"], return_arrays=True, **kw)
        # the restated selection is numpy's own on this host
        assert np.array_equal(ia, _np_select(s32, c["k"], kw)), name
        _, ic, wc = R.route_topk_canonical(s32, c["k"], return_arrays=True, **kw)
        ties = R.boundary_ties(s32, c["k"], scoring=c["scoring"], e_score_bias=bias,
                               n_group=c.get("n_group", 0), topk_group=c.get("topk_group", 0))
        np.savez_compressed(os.path.join(HERE, f"route_{name}.npz"), logits=logits,
                            bias=bias if bias is not None else np.zeros(0, np.float32),
                            top_k=c["k"], norm=int(c["norm"]), scoring=c["scoring"],
                            scale=np.float32(c.get("scale", 1.0)), n_group=c.get("n_group", 0),
                            topk_group=c.get("topk_group", 0), idx_argpartition=ia.astype(np.int32),
                            w_argpartition=wa, idx_canonical=ic.astype(np.int32), w_canonical=wc,
                            boundary_ties=ties)
        print(name, "ties:", int(ties.sum()))


def _np_select(s32, k, kw):
    """The reference's selection with the installed np.argpartition
    (fastllm_py/expert_router.py:36-55, same float32 arithmetic as the oracle)."""
    probs, select = R._scores(s32, kw["scoring"], kw["e_score_bias"])
    ng, tg = kw["n_group"], kw["topk_group"]
    if ng and ng > 1 and 0 < tg < ng:
        T, E = select.shape
        gs = select.reshape(T, ng, E // ng)
        group_score = np.sort(gs, axis=-1)[:, :, -min(2, E // ng):].sum(-1)
        keep = np.argpartition(-group_score, tg - 1, axis=-1)[:, :tg]
        masked = np.ones((T, ng), dtype=bool)
        np.put_along_axis(masked, keep, False, axis=-1)
        select = np.where(np.repeat(masked, E // ng, axis=1), np.float32(-np.inf), select)
    return np.argpartition(-select, k - 1, axis=-1)[:, :k]


def packers():
    rng = np.random.default_rng(77)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    p3, s3, z3 = Q.quantize_int4_group(w, 128)
    q9, s9, z9 = Q.quantize_int4_marlin(w, 128)
    s9p, z9p = Q.marlin_scales_zeros(s9, z9)
    p13, s13, z13 = Q.quantize_int4_rowmajor(w.astype(np.float16), 128)
    wf = (rng.standard_normal((130, 200)) * 3).astype(np.float32)
    q8, s8 = Q.quantize_fp8_block(wf, 128)
    np.savez_compressed(os.path.join(HERE, "packers.npz"), w=w, group_packed=p3, group_scales=s3,
                        group_zeros=z3, marlin_q=q9, marlin_gptq=Q.pack_gptq(q9),
                        marlin_scales=s9p, marlin_zeros=z9p, rowmajor_packed=p13,
                        rowmajor_scales=s13, rowmajor_zeros=z13, fp8_w=wf, fp8_q=q8, fp8_scales=s8)


if __name__ == "__main__":
    routing()
    packers()

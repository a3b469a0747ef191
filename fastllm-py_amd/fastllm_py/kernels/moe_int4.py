"""Row-major INT4 group-quant GEMV, gate matvec and the fused selective MoE FFN.

Drop-in for the reference's ``fastllm_py/kernels/moe_int4.py`` (lines 1-506)
and the hot-path kernels of ``fastllm_py/graph_decode.py`` (``_dgemv``
:748-765, ``_route_topk_kernel`` :242-285, ``_moe_branch`` :669-700), with
PyTorch-ROCm tensors as buffers and gfx950 HIP kernels (csrc/moe_int4.hip,
csrc/packers.hip) doing the work.

Format for a weight W of shape (out, in), group size gs along ``in``:
  qweight : (out, in//2) uint8   -- two int4 nibbles/byte, even col in low nibble
  scales  : (out, in//gs) fp16
  zeros   : (out, in//gs) fp16   -- dequant(W[o,i]) = (q - zero) * scale

The fused MoE keeps its stacked experts in a tile layout of its own
(``build_stacked_experts`` / ``tile_pack``; ``unpack_stacked`` inverts it)
so every wave load reads one contiguous 1 KB block.  Activations feed the
matrix cores as fp16.
"""
from __future__ import annotations

import numpy as np

from .. import _native as nat


# ----------------------------------------------------------------- packers
def _rowmajor_device(W, group_size):
    """(..., out, in) float -> (qweight, scales, zeros) device tensors."""
    t = nat.torch()
    w = nat.to_device(W, t.float32)
    lead = tuple(w.shape[:-2])
    out_f, in_f = w.shape[-2:]
    assert in_f % group_size == 0 and in_f % 2 == 0
    batch = int(np.prod(lead)) if lead else 1
    qw = t.empty(lead + (out_f, in_f // 2), dtype=t.uint8, device=w.device)
    sc = t.empty(lead + (out_f, in_f // group_size), dtype=t.float16, device=w.device)
    ze = t.empty_like(sc)
    rc = nat.lib().fastllm_quantize_int4_rowmajor(nat.ptr(w), nat.ptr(qw), nat.ptr(sc),
                                                  nat.ptr(ze), batch, out_f, in_f, group_size,
                                                  nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_quantize_int4_rowmajor")
    return qw, sc, ze


def quantize_int4_rowmajor(w, group_size: int = 128, xp=np) -> dict:
    """RTN group INT4, row-major (moe_int4.py:24-40).  numpy in -> numpy arrays
    out (computed on the GPU); torch in -> device tensors."""
    numpy_in = nat.host_out(w, xp)
    qw, sc, ze = _rowmajor_device(np.asarray(w) if numpy_in else w, group_size)
    out_f, in_f = qw.shape[0], qw.shape[1] * 2
    return {"qweight": nat.as_output(qw, numpy_in), "scales": nat.as_output(sc, numpy_in),
            "zeros": nat.as_output(ze, numpy_in), "shape": (out_f, in_f), "group": group_size}


def dequantize_int4_rowmajor(payload, xp=np):
    """(q - zero) * scale -> fp32 (moe_int4.py:43-54)."""
    t = nat.torch()
    numpy_in = nat.host_out(payload["qweight"], xp)
    qw = nat.to_device(payload["qweight"], t.uint8)
    sc = nat.to_device(payload["scales"], t.float16)
    ze = nat.to_device(payload["zeros"], t.float16)
    out_f, in_f = payload["shape"]
    batch = qw.numel() // (out_f * (in_f // 2))
    out = t.empty(tuple(qw.shape[:-2]) + (out_f, in_f), dtype=t.float32, device=qw.device)
    rc = nat.lib().fastllm_dequantize_int4_rowmajor(nat.ptr(qw), nat.ptr(sc), nat.ptr(ze),
                                                    nat.ptr(out), batch, out_f, in_f,
                                                    payload["group"], nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_dequantize_int4_rowmajor")
    return nat.as_output(out, numpy_in)


def _quantize_int4_rowmajor_batched(W, group_size: int, xp=np):
    """(E, out, in) -> (qweight (E,out,in/2), scales, zeros, (out,in))
    (moe_int4.py:97-113), one GPU launch for all E."""
    qw, sc, ze = _rowmajor_device(W, group_size)
    return qw, sc, ze, (qw.shape[-2], qw.shape[-1] * 2)


def tile_pack(qweight, scales, zeros, group_size: int):
    """Row-major INT4 (rows, in/2) u8 + (rows, in/gs) fp16 scales/zeros (any
    leading dims, rows % 16 == 0) -> the fused MoE's tile layout:
    qtile (rows/16, in/128, 1024) u8 and sz (rows/16, in/gs, 16) int32 holding
    scale bits | zero bits << 16 (csrc/moe_int4.hip describes the layout)."""
    t = nat.torch()
    q = nat.to_device(qweight, t.uint8).contiguous()
    sc = nat.to_device(scales, t.float16).contiguous()
    ze = nat.to_device(zeros, t.float16).contiguous()
    in_f = q.shape[-1] * 2
    rows = q.numel() // (in_f // 2)
    qt = t.empty((rows // 16, in_f // 128, 1024), dtype=t.uint8, device=q.device)
    sz = t.empty((rows // 16, in_f // group_size, 16), dtype=t.int32, device=q.device)
    rc = nat.lib().fastllm_moe_int4_tile_repack(nat.ptr(q), nat.ptr(sc), nat.ptr(ze), nat.ptr(qt),
                                                nat.ptr(sz), rows, in_f, group_size,
                                                nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_moe_int4_tile_repack")
    return qt, sz


def tile_unpack(qtile, sz, rows: int, in_f: int, group_size: int):
    """Inverse of ``tile_pack`` -> (qweight (rows, in/2) u8, scales, zeros
    (rows, in/gs) fp16) device tensors, bit-exact."""
    t = nat.torch()
    q = t.empty((rows, in_f // 2), dtype=t.uint8, device=qtile.device)
    sc = t.empty((rows, in_f // group_size), dtype=t.float16, device=qtile.device)
    ze = t.empty_like(sc)
    rc = nat.lib().fastllm_moe_int4_tile_unpack(nat.ptr(qtile), nat.ptr(sz), nat.ptr(q),
                                                nat.ptr(sc), nat.ptr(ze), rows, in_f, group_size,
                                                nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_moe_int4_tile_unpack")
    return q, sc, ze


def build_stacked_experts(expert_ws, group_size: int = 128, xp=np) -> dict:
    """Stack E experts' {gate, up, down}, quantize them (row-major RTN group
    INT4, moe_int4.py:116-133) and store them in the fused MoE's tile layout,
    indexable by expert id: ``{proj}.qtile`` (E, out/16, in/128, 1024) u8,
    ``{proj}.sz`` (E, out/16, in/gs, 16) int32, ``{proj}.shape`` (out, in).
    The reference's callers only hand this dict to the fused MoE kernels;
    ``unpack_stacked`` recovers the row-major payload."""
    t = nat.torch()
    out = {"group": group_size, "layout": "tile16x128"}
    for proj in ("gate", "up", "down"):
        ws = [w[proj] for w in expert_ws]
        if nat.is_tensor(ws[0]):
            stack = t.stack([nat.to_device(w) for w in ws])
        else:
            stack = np.stack([np.asarray(w) for w in ws])
        qw, sc, ze, shp = _quantize_int4_rowmajor_batched(stack, group_size)
        out.update(stack_tiles(proj, qw, sc, ze, group_size))
    return out


def stack_marlin_experts(payloads, group_size: int = 128) -> dict:
    """Stacked experts straight from resident Marlin payloads: ``payloads`` is
    a list over experts of {"gate", "up", "down"} -> Marlin dicts (qweight,
    scales, zeros, as ``moe.quantize_marlin_matrix_device`` makes them).  Each
    matrix is copied on the GPU into its expert's slot of the tile layout with
    its own integers, scales and zeros -- no fp16 round trip and no
    requantization (the reference dequantizes to fp16 and quantizes again,
    moe_int4.py:116-133; docs/next-optimizations.md:108-135)."""
    t = nat.torch()
    out = {"group": group_size, "layout": "tile16x128"}
    E = len(payloads)
    hs = nat.current_stream_handle()
    for proj in ("gate", "up", "down"):
        p0 = payloads[0][proj]
        out_f = p0["scales"].shape[1]
        G = p0["scales"].shape[0]
        in_f = G * group_size
        dev = p0["qweight"].device
        qt = t.empty((E, out_f // 16, in_f // 128, 1024), dtype=t.uint8, device=dev)
        sz = t.empty((E, out_f // 16, G, 16), dtype=t.int32, device=dev)
        for e, pe in enumerate(payloads):
            p = pe[proj]
            if tuple(p["scales"].shape) != (G, out_f):
                raise ValueError(f"stack_marlin_experts: expert {e} {proj} scales {tuple(p['scales'].shape)}")
            rc = nat.lib().fastllm_marlin_to_moe_tile(nat.ptr(p["qweight"]), nat.ptr(p["scales"]),
                                                      nat.ptr(p["zeros"]), nat.ptr(qt[e]), nat.ptr(sz[e]),
                                                      out_f, in_f, group_size, hs)
            nat.check_rc(rc, "fastllm_marlin_to_moe_tile")
        out[f"{proj}.qtile"], out[f"{proj}.sz"], out[f"{proj}.shape"] = qt, sz, (out_f, in_f)
    return out


def stack_tiles(proj: str, qw, sc, ze, group_size: int) -> dict:
    """Row-major stacked (E, out, in/2) / (E, out, in/gs) -> the tile-layout
    entries of one projection of a stacked-experts dict."""
    E, out_f, half = qw.shape
    qt, sz = tile_pack(qw, sc, ze, group_size)
    return {f"{proj}.qtile": qt.reshape(E, out_f // 16, half * 2 // 128, 1024),
            f"{proj}.sz": sz.reshape(E, out_f // 16, half * 2 // group_size, 16),
            f"{proj}.shape": (out_f, half * 2)}


# low-precision expert formats of the fused MoE: name -> (C format code, group)
LOWP_FORMATS = {"fp8": (1, 128), "mxfp4": (2, 32)}


def stack_lowp(fmt: str, proj: str, W) -> dict:
    """One projection of E stacked experts, W (E, out, in) float (device
    tensor or numpy), quantized on the GPU and stored in the fused MoE's
    low-precision tile layout:

    * ``fp8``: 128x128-block e4m3 (quantize_fp8_block's format,
      quantizer.py:65-85; out % 128 == 0 so no block spans two experts):
      ``{proj}.qtile`` (E, out/16, in/128, 2048) u8, ``{proj}.sz`` the fp32
      block scales (E, out/128, in/128);
    * ``mxfp4``: OCP MXFP4 (quantizer.quantize_mxfp4): ``{proj}.qtile``
      (E, out/16, in/128, 1024) u8, ``{proj}.sz`` (E, out/16, in/128, 16)
      int32 words of four E8M0 scales.

    Also ``{proj}.shape`` (out, in)."""
    t = nat.torch()
    if fmt not in LOWP_FORMATS:
        raise ValueError(f"stack_lowp: unknown format {fmt!r} (fp8, mxfp4)")
    wd = nat.to_device(W, t.float32).contiguous()
    E, out_f, in_f = wd.shape
    if out_f % 128 or in_f % 128:
        raise ValueError(f"stack_lowp: out {out_f} and in {in_f} must be multiples of 128")
    rows = E * out_f
    w2 = wd.reshape(rows, in_f)
    hs = nat.current_stream_handle()
    lib = nat.lib()
    qt = t.empty((E, out_f // 16, in_f // 128, 2048 if fmt == "fp8" else 1024), dtype=t.uint8,
                 device=wd.device)
    if fmt == "fp8":
        q = t.empty((rows, in_f), dtype=t.uint8, device=wd.device)
        sz = t.empty((E, out_f // 128, in_f // 128), dtype=t.float32, device=wd.device)
        nat.check_rc(lib.fastllm_quantize_fp8_block(nat.ptr(w2), nat.ptr(q), nat.ptr(sz), rows, in_f,
                                                    128, hs), "fastllm_quantize_fp8_block")
        nat.check_rc(lib.fastllm_moe_fp8_tile_repack(nat.ptr(q), nat.ptr(qt), rows, in_f, hs),
                     "fastllm_moe_fp8_tile_repack")
    else:
        codes = t.empty((rows, in_f // 2), dtype=t.uint8, device=wd.device)
        e8 = t.empty((rows, in_f // 32), dtype=t.uint8, device=wd.device)
        sz = t.empty((E, out_f // 16, in_f // 128, 16), dtype=t.int32, device=wd.device)
        nat.check_rc(lib.fastllm_quantize_mxfp4(nat.ptr(w2), nat.ptr(codes), nat.ptr(e8), rows, in_f,
                                                hs), "fastllm_quantize_mxfp4")
        nat.check_rc(lib.fastllm_moe_mxfp4_tile_repack(nat.ptr(codes), nat.ptr(e8), nat.ptr(qt),
                                                       nat.ptr(sz), rows, in_f, hs),
                     "fastllm_moe_mxfp4_tile_repack")
    return {f"{proj}.qtile": qt, f"{proj}.sz": sz, f"{proj}.shape": (out_f, in_f)}


def build_stacked_experts_lowp(expert_ws, fmt: str) -> dict:
    """``build_stacked_experts`` with FP8 (128x128 block e4m3) or MXFP4
    expert weights: the tensor-core fused-MoE variant of
    docs/next-optimizations.md:160-184.  ``expert_ws`` is a list over
    experts of {"gate", "up", "down"} float weights (out, in).  The dict
    goes to moe_forward / moe_route_forward like the INT4 one."""
    t = nat.torch()
    code, group = LOWP_FORMATS.get(fmt, (None, None))
    if code is None:
        raise ValueError(f"build_stacked_experts_lowp: unknown format {fmt!r} (fp8, mxfp4)")
    out = {"group": group, "format": fmt, "layout": "tile16x128"}
    for proj in ("gate", "up", "down"):
        ws = [w[proj] for w in expert_ws]
        stack = (t.stack([nat.to_device(w, t.float32) for w in ws]) if nat.is_tensor(ws[0])
                 else np.stack([np.asarray(w, np.float32) for w in ws]))
        out.update(stack_lowp(fmt, proj, stack))
    return out


def _format_code(stacked, shared=None) -> int:
    """0 for INT4 stacks, else the low-precision format code (shared expert
    in the same format)."""
    fmt = stacked.get("format", "int4")
    sfmt = shared.get("format", "int4") if shared is not None else fmt
    if sfmt != fmt:
        raise ValueError(f"fused MoE: routed experts are {fmt}, the shared expert {sfmt}")
    if fmt == "int4":
        return 0
    if fmt not in LOWP_FORMATS:
        raise ValueError(f"fused MoE: unknown expert format {fmt!r}")
    return LOWP_FORMATS[fmt][0]


def unpack_stacked(stacked) -> dict:
    """Tile-layout stacked experts -> row-major {proj}.qweight (E, out, in/2)
    u8, {proj}.scales / {proj}.zeros (E, out, in/gs) fp16 device tensors."""
    gs = stacked["group"]
    out = {"group": gs}
    for proj in ("gate", "up", "down"):
        qt = stacked[f"{proj}.qtile"]
        out_f, in_f = stacked[f"{proj}.shape"]
        E = qt.shape[0]
        q, sc, ze = tile_unpack(qt, stacked[f"{proj}.sz"], E * out_f, in_f, gs)
        out[f"{proj}.qweight"] = q.reshape(E, out_f, in_f // 2)
        out[f"{proj}.scales"] = sc.reshape(E, out_f, in_f // gs)
        out[f"{proj}.zeros"] = ze.reshape(E, out_f, in_f // gs)
        out[f"{proj}.shape"] = (out_f, in_f)
    return out


# ------------------------------------------------------------------ GEMVs
def _rm_gemv(x, payload, out, y_dtype):
    t = nat.torch()
    out_f, in_f = payload["shape"]
    x = nat.to_device(x)
    if x.dtype not in (t.float32, t.float16):
        x = x.to(t.float32)
    x2 = x.reshape(-1, in_f)
    M = x2.shape[0]
    y = out if out is not None else t.empty((M, out_f), dtype=y_dtype, device=x.device)
    rc = nat.lib().fastllm_int4_rowmajor_gemv(
        nat.ptr(x2), 1 if x2.dtype == t.float32 else 0, nat.ptr(payload["qweight"]),
        nat.ptr(payload["scales"]), nat.ptr(payload["zeros"]), nat.ptr(y),
        1 if y.dtype == t.float32 else 0, M, out_f, in_f, payload["group"],
        nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_int4_rowmajor_gemv")
    return y


def gemv_int4(x, payload, out=None):
    """y = x @ dequant(W).T for decode rows (moe_int4.py:490-506).  x (in,) or
    (M, in) fp32 -> fp32 (out,) / (M, out)."""
    t = nat.torch()
    y = _rm_gemv(x, payload, out, t.float32)
    return y.reshape(-1) if (nat.to_device(x).dim() == 1 and out is None) else y


def dgemv(x, payload, out=None):
    """graph_decode._dgemv (graph_decode.py:748-765): x (1, in) or (in,) fp16 or
    fp32 -> same dtype (1, out), written into ``out`` when given."""
    t = nat.torch()
    xd = nat.to_device(x)
    y = _rm_gemv(xd, payload, out, xd.dtype if xd.dtype in (t.float16, t.float32) else t.float32)
    return y.reshape(1, -1)


def gate_matvec(x, gate_w, E, hidden, out=None, threads=128):
    """logits (E,) = x (hidden,) @ gate_w (E, hidden).T in fp32 (moe_int4.py:162-169).
    x may also be (T, hidden) -> (T, E)."""
    t = nat.torch()
    xd = nat.to_device(x, t.float32)
    x2 = xd.reshape(-1, hidden)
    T = x2.shape[0]
    gw = nat.to_device(gate_w, t.float16)
    y = out if out is not None else t.empty((T, E) if xd.dim() > 1 else (E,), dtype=t.float32,
                                            device=xd.device)
    rc = nat.lib().fastllm_gate_matvec(nat.ptr(x2), nat.ptr(gw), None, nat.ptr(y), None, T, E,
                                       hidden, nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_gate_matvec")
    return y


# -------------------------------------------------------------- fused MoE
def _stacked_ptrs(st):
    return [nat.ptr(st[f"{p}.{k}"]) for p in ("gate", "up", "down") for k in ("qtile", "sz")]


# call flags of the fused MoE entries (fastllm_moe_fused_ex / _routed_ex)
MOE_DETERMINISTIC = 1


def moe_workspace_bytes(T: int, hidden: int, inter: int, shared_inter: int,
                        max_entries: int, deterministic: bool = False) -> int:
    """Device workspace (bytes) of one fused MoE call of this shape (with the
    deterministic combine's term rows when ``deterministic``)."""
    if deterministic:
        n = nat.lib().fastllm_moe_workspace_bytes_ex(T, hidden, inter, shared_inter or 0,
                                                     max_entries, MOE_DETERMINISTIC)
    else:
        n = nat.lib().fastllm_moe_int4_workspace_bytes(T, hidden, inter, shared_inter or 0,
                                                       max_entries)
    if n == 0:
        raise ValueError(f"unsupported fused MoE shape T={T} hidden={hidden} inter={inter} "
                         f"shared_inter={shared_inter}")
    return int(n)


def build_lists(T: int, E: int, *, rw=None, slot_coef=None, cand=None, out=None,
                stream=None) -> dict:
    """Expert-major MoE lists for the fused MoE from dense weights ``rw``
    (T, E) (slots = ``cand`` experts, or all E in order) or per-slot weights
    ``slot_coef`` (S, T) for the experts ``cand`` (S,).  Entries with weight 0
    are dropped.  Same layout as the router's lists."""
    t = nat.torch()
    if slot_coef is not None:
        coef = nat.to_device(slot_coef, t.float32).contiguous()
        S = coef.shape[0]
        dev = coef.device
        rwd = None
    else:
        rwd = nat.to_device(rw, t.float32).reshape(T, E).contiguous()
        coef = None
        dev = rwd.device
    cd = None
    if cand is not None:
        cd = nat.to_device(cand, t.int32).reshape(-1).contiguous()
        S = cd.numel()
    elif slot_coef is None:
        S = E
    o = out if out is not None else {}

    def buf(name, shape, dtype):
        if name not in o:
            o[name] = t.empty(shape, dtype=dtype, device=dev)
        return o[name]

    na = buf("n_active", (1,), t.int32)
    act = buf("active", (S,), t.int32)
    offs = buf("offsets", (S + 1,), t.int32)
    tok = buf("tok", (S * T,), t.int32)
    tokw = buf("tokw", (S * T,), t.float32)
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    rc = nat.lib().fastllm_moe_build_lists(
        nat.ptr(rwd) if rwd is not None else None, nat.ptr(coef) if coef is not None else None,
        nat.ptr(cd) if cd is not None else None, T, E, S, nat.ptr(na), nat.ptr(act),
        nat.ptr(offs), nat.ptr(tok), nat.ptr(tokw), h)
    nat.check_rc(rc, "fastllm_moe_build_lists")
    return o


def moe_forward(x, stacked, E, hidden, inter, lists, *, max_slots=None, max_entries=None,
                shared=None, shared_inter=0, shared_coef=None, out=None, workspace=None,
                stream=None, deterministic=False):
    """Fused selective INT4 MoE FFN (x (T, hidden) fp32):

    y[t] = sum_{entries p of t} tokw[p] * down_e(silu(gate_e x_t) * up_e x_t)
           + shared_coef[t] * shared(x_t)

    ``lists`` are expert-major MoE lists (``route_topk_device`` or
    ``build_lists``).  Gate/up run only over the tokens routed to each
    expert; the down projection adds each expert's term into y with fp32
    atomics, as the reference's moew_down does, so the last bits depend on
    arrival order -- unless ``deterministic``: then the terms go to the
    workspace and one more launch sums each token's terms in a fixed order
    (ascending expert, then the shared expert), so repeated calls give
    bit-identical y.  Up to 16 tokens take the decode kernels (weights split
    over the waves along k); more tokens take the grouped GEMM kernels (each
    slot's entries in 64-row chunks on the matrix cores), the prefill form of
    MoELayer._run_gpu_experts (fastllm_py/moe.py:135-159).  ``workspace``
    (uint8 device tensor) is reused when large enough, else allocated."""
    t = nat.torch()
    xd = nat.to_device(x, t.float32)
    x2 = xd.reshape(-1, hidden).contiguous()
    T = x2.shape[0]
    if max_entries is None:
        max_entries = lists["tok"].numel()
    if max_slots is None:
        max_slots = min(lists["active"].numel(), max_entries)
    sint = int(shared_inter or 0) if shared is not None else 0
    need = moe_workspace_bytes(T, hidden, inter, sint, max_entries, deterministic)
    ws = workspace
    if ws is None or ws.numel() * ws.element_size() < need or not ws.is_contiguous():
        ws = t.empty((need,), dtype=t.uint8, device=xd.device)
    y = out if out is not None else t.empty((T, hidden), dtype=t.float32, device=xd.device)
    sp = _stacked_ptrs(shared) if shared is not None else [None] * 6
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    code = _format_code(stacked, shared)
    args = [nat.ptr(x2), T, hidden, stacked["group"], E, inter, *_stacked_ptrs(stacked), sint, *sp,
            nat.ptr(shared_coef) if shared_coef is not None else None,
            nat.ptr(lists["n_active"]), nat.ptr(lists["active"]), nat.ptr(lists["offsets"]),
            nat.ptr(lists["tok"]), nat.ptr(lists["tokw"]), int(max_slots), int(max_entries),
            nat.ptr(ws), ws.numel() * ws.element_size(), nat.ptr(y), h]
    if deterministic:
        nat.check_rc(nat.lib().fastllm_moe_fused_ex(code, MOE_DETERMINISTIC, *args),
                     "fastllm_moe_fused_ex")
    elif code:
        nat.check_rc(nat.lib().fastllm_moe_lowp_fused(code, *args), "fastllm_moe_lowp_fused")
    else:
        nat.check_rc(nat.lib().fastllm_moe_int4_fused(*args), "fastllm_moe_int4_fused")
    return y


def moe_route_forward(x, logits, stacked, top_k, E, hidden, inter, *, norm_topk_prob=False,
                      scoring="softmax", routed_scaling=1.0, e_score_bias=None, n_group=0,
                      topk_group=0, shared=None, shared_inter=0, shared_logit=None, route=None,
                      out=None, workspace=None, stream=None, deterministic=False):
    """Router + fused MoE in one native call: routes ``logits`` (T, E)
    exactly like ``route_topk_device`` (same keyword meaning, same outputs,
    which land in ``route``: topk_ids, topk_w, rw, lists, shared_coef) and
    returns y (T, hidden) fp32 = moe_forward over those lists
    (graph_decode._moe_branch, graph_decode.py:669-700).  Up to 16 tokens
    the decode kernels; above, the router's last workgroup builds the lists
    and the grouped GEMMs follow (three launches), which keeps an arrival
    counter in the workspace: a ``workspace`` passed in must have been
    zero-filled before its first use (calls leave the counter at zero).
    ``route`` / ``workspace`` / ``out`` may carry persistent buffers for
    graph capture.  ``deterministic``: the ordered combine of moe_forward
    (bit-identical repeats, one more launch)."""
    t = nat.torch()
    xd = nat.to_device(x, t.float32)
    x2 = xd.reshape(-1, hidden).contiguous()
    T = x2.shape[0]
    s = nat.to_device(logits)
    if s.dtype != t.float32:
        s = s.to(t.float32)
    s = s.reshape(T, E).contiguous()
    dev = x2.device
    o = route if route is not None else {}

    def buf(name, shape, dtype):
        if name not in o:
            o[name] = t.empty(shape, dtype=dtype, device=dev)
        return o[name]

    ids = buf("topk_ids", (T, top_k), t.int32)
    w = buf("topk_w", (T, top_k), t.float32)
    rw = buf("rw", (T, E), t.float32)
    na = buf("n_active", (1,), t.int32)
    act = buf("active", (E,), t.int32)
    offs = buf("offsets", (E + 1,), t.int32)
    tok = buf("tok", (T * top_k,), t.int32)
    tokw = buf("tokw", (T * top_k,), t.float32)
    bias = None
    if scoring == "sigmoid" and e_score_bias is not None:
        bias = nat.to_device(e_score_bias, t.float32)
    sl = sc = None
    if shared_logit is not None:
        sl = nat.to_device(shared_logit, t.float32).reshape(-1)
        sc = buf("shared_coef", (T,), t.float32)
    sint = int(shared_inter or 0) if shared is not None else 0
    need = moe_workspace_bytes(T, hidden, inter, sint, T * top_k, deterministic)
    ws = workspace
    if ws is None or ws.numel() * ws.element_size() < need or not ws.is_contiguous():
        ws = t.zeros((need,), dtype=t.uint8, device=dev)  # zero: the router's counter
    y = out if out is not None else t.empty((T, hidden), dtype=t.float32, device=dev)
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    args = _routed_args(s, top_k, scoring, norm_topk_prob, routed_scaling, bias, n_group,
                        topk_group, sl, o, x2, T, hidden, stacked, E, inter, shared, sint)
    code = _format_code(stacked, shared)
    if deterministic:
        rc = nat.lib().fastllm_moe_routed_ex(code, MOE_DETERMINISTIC, *args, nat.ptr(ws),
                                             ws.numel() * ws.element_size(), nat.ptr(y), h)
        nat.check_rc(rc, "fastllm_moe_routed_ex")
    elif code:
        rc = nat.lib().fastllm_moe_lowp_routed(code, *args, nat.ptr(ws), ws.numel() * ws.element_size(),
                                               nat.ptr(y), h)
        nat.check_rc(rc, "fastllm_moe_lowp_routed")
    else:
        rc = nat.lib().fastllm_moe_int4_routed(*args, nat.ptr(ws), ws.numel() * ws.element_size(),
                                               nat.ptr(y), h)
        nat.check_rc(rc, "fastllm_moe_int4_routed")
    return y


def _routed_args(s, top_k, scoring, norm_topk_prob, routed_scaling, bias, n_group, topk_group,
                 sl, o, x2, T, hidden, stacked, E, inter, shared, sint):
    """Arguments of the routed MoE entries up to the workspace."""
    sp = _stacked_ptrs(shared) if shared is not None else [None] * 6
    sc = o.get("shared_coef") if sl is not None else None
    return [nat.ptr(s), int(top_k), 1 if scoring == "sigmoid" else 0, 1 if norm_topk_prob else 0,
            float(routed_scaling), nat.ptr(bias) if bias is not None else None, int(n_group or 0),
            int(topk_group or 0), nat.ptr(sl) if sl is not None else None,
            nat.ptr(o["topk_ids"]), nat.ptr(o["topk_w"]), nat.ptr(o["rw"]),
            nat.ptr(sc) if sc is not None else None, nat.ptr(o["n_active"]),
            nat.ptr(o["active"]), nat.ptr(o["offsets"]), nat.ptr(o["tok"]), nat.ptr(o["tokw"]),
            nat.ptr(x2), T, hidden, stacked["group"], E, inter, *_stacked_ptrs(stacked), sint, *sp]


# sizes (elements, dtype name) of the router outputs of T tokens, top_k of E
def _route_buffer_shapes(T, E, top_k):
    return {"topk_ids": ((T, top_k), "int32"), "topk_w": ((T, top_k), "float32"),
            "rw": ((T, E), "float32"), "n_active": ((1,), "int32"), "active": ((E,), "int32"),
            "offsets": ((E + 1,), "int32"), "tok": ((T * top_k,), "int32"),
            "tokw": ((T * top_k,), "float32"), "shared_coef": ((T,), "float32")}


def alloc_route_buffers(T: int, E: int, top_k: int, device="cuda") -> dict:
    """Persistent router-output buffers for ``moe_route_forward`` /
    ``moe_route_forward_noalloc`` (allocated once, outside any loop that must
    not allocate)."""
    t = nat.torch()
    return {k: t.empty(shape, dtype=getattr(t, dt), device=device)
            for k, (shape, dt) in _route_buffer_shapes(T, E, top_k).items()}


def moe_route_forward_noalloc(x, logits, stacked, top_k, E, hidden, inter, *, route, out,
                              norm_topk_prob=False, scoring="softmax", routed_scaling=1.0,
                              e_score_bias=None, n_group=0, topk_group=0, shared=None,
                              shared_inter=0, shared_logit=None, stream=None):
    """``moe_route_forward`` through fastllm_moe_int4_routed_noalloc: the
    workspace is the library's static per-GPU scratch (16 MiB), so nothing is
    allocated, by this wrapper either.  Every buffer must be supplied: x
    (T, hidden) and logits (T, E) contiguous fp32 device tensors, ``route``
    from ``alloc_route_buffers``, ``out`` (T, hidden) fp32.  Calls that
    overlap on one GPU share the scratch and race.  Raises ValueError for
    missing or wrongly typed buffers and for shapes whose workspace exceeds
    the scratch."""
    t = nat.torch()
    for name, v in (("x", x), ("logits", logits), ("out", out)):
        if not isinstance(v, t.Tensor) or v.dtype != t.float32 or not v.is_cuda \
                or not v.is_contiguous():
            raise ValueError(f"moe_route_forward_noalloc: {name} must be a contiguous fp32 "
                             f"device tensor")
    T = x.numel() // hidden
    if T < 1 or x.numel() != T * hidden or logits.numel() != T * E or out.numel() != T * hidden:
        raise ValueError("moe_route_forward_noalloc: x (T, hidden), logits (T, E) and out "
                         "(T, hidden)")
    # the optional per-token / per-expert vectors reach the kernel as raw
    # pointers too: same checks, with their lengths
    for name, v, n in (("shared_logit", shared_logit, T), ("e_score_bias", e_score_bias, E)):
        if v is None:
            continue
        if not isinstance(v, t.Tensor) or v.dtype != t.float32 or not v.is_cuda \
                or not v.is_contiguous() or v.numel() != n:
            raise ValueError(f"moe_route_forward_noalloc: {name} must be a contiguous fp32 "
                             f"device tensor of {n} elements")
        if v.device != x.device:
            raise ValueError(f"moe_route_forward_noalloc: {name} must live on {x.device}")
    for k, (shape, dt) in _route_buffer_shapes(T, E, top_k).items():
        if k == "shared_coef" and shared_logit is None:
            continue
        buf = route.get(k)
        n = 1
        for d in shape:
            n *= d
        if buf is None or buf.dtype != getattr(t, dt) or not buf.is_contiguous() \
                or buf.numel() < n:
            raise ValueError(f"moe_route_forward_noalloc: route[{k!r}] must hold {n} {dt}")
    if _format_code(stacked, shared):
        raise ValueError("moe_route_forward_noalloc: INT4 experts only (FP8 / MXFP4 experts take "
                         "moe_route_forward)")
    bias = None
    if scoring == "sigmoid" and e_score_bias is not None:
        bias = e_score_bias
    sint = int(shared_inter or 0) if shared is not None else 0
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    args = _routed_args(logits, top_k, scoring, norm_topk_prob, routed_scaling, bias, n_group,
                        topk_group, shared_logit, route, x, T, hidden, stacked, E, inter, shared,
                        sint)
    rc = nat.lib().fastllm_moe_int4_routed_noalloc(*args, nat.ptr(out), h)
    if rc == 1:
        raise ValueError(f"moe_route_forward_noalloc: arguments or shape refused (T={T} "
                         f"hidden={hidden} inter={inter} shared_inter={sint}; a workspace above "
                         f"the 16 MiB static scratch takes moe_route_forward)")
    nat.check_rc(rc, "fastllm_moe_int4_routed_noalloc")
    return out


def fused_moe_weighted(x, stacked, rw, E, hidden, inter, out=None, inter_buf=None,
                       threads=256, rpb=8, aidx=None):
    """(E,)-routing-weight-driven selective MoE FFN (moe_int4.py:263-294):
    y (hidden,) = sum_{e: rw[e] > 0} rw[e] * FFN_e(x).  ``aidx`` (K,) lists the
    active experts; without it every expert is scanned and those with zero
    weight are skipped.  ``inter_buf`` may be a reusable uint8 workspace."""
    t = nat.torch()
    rwd = nat.to_device(rw, t.float32).reshape(1, -1)
    cand = None if aidx is None else nat.to_device(aidx, t.int32).reshape(-1)
    L = build_lists(1, E, rw=rwd, cand=cand)
    y = out.reshape(1, hidden) if out is not None else None
    r = moe_forward(x, stacked, E, hidden, inter, L, out=y, workspace=inter_buf)
    return r.reshape(hidden)


def fused_moe_ffn2(x, stacked, eidx, rw, hidden, inter, out=None, inter_buf=None, threads=128):
    """Index-driven selective MoE FFN (moe_int4.py:372-396):
    y = sum_k rw[k] * FFN_{eidx[k]}(x)."""
    t = nat.torch()
    cand = nat.to_device(eidx, t.int32).reshape(-1)
    coef = nat.to_device(rw, t.float32).reshape(-1, 1).contiguous()
    E = stacked["gate.qtile"].shape[0]
    L = build_lists(1, E, slot_coef=coef, cand=cand)
    y = out.reshape(1, hidden) if out is not None else None
    r = moe_forward(x, stacked, E, hidden, inter, L, out=y, workspace=inter_buf)
    return r.reshape(hidden)


def fused_moe_ffn(x, stacked, eidx, rw, hidden, inter, out=None):
    """One-launch-per-expert variant in the reference (moe_int4.py:466-487);
    same math, same kernels here."""
    return fused_moe_ffn2(x, stacked, eidx, rw, hidden, inter, out=out)


# ------------------------------------------------------- graph decode branch
def route_topk_gpu(logits, top_k, *, norm=False, scale=1.0, rw=None, aidx=None):
    """graph_decode._route_topk_kernel (graph_decode.py:242-285) for one token:
    writes the (E,) weight vector and the (K,) active expert list.  Selection
    and weights are numpy-exact (the reference kernel's __expf is not)."""
    from ..expert_router import route_topk_device

    r = route_topk_device(logits, top_k, norm_topk_prob=norm, routed_scaling=scale)
    if rw is not None:
        rw.copy_(r["rw"].reshape(rw.shape))
    if aidx is not None:
        aidx.copy_(r["topk_ids"].reshape(aidx.shape))
    return r


def moe_branch(x, gate_w, stacked, top_k, *, E, hidden, inter, norm=False, scale=1.0,
               shared=None, shared_inter=0, shared_gate_w=None, bufs=None, stream=None):
    """One fused MoE layer, all on the device with no host sync
    (graph_decode._moe_branch, graph_decode.py:669-700): gate matvec (+
    shared gate) -> router -> fused routed + shared FFN (one native call).
    Returns (T, hidden) fp32.  ``bufs`` may carry persistent buffers for
    graph capture (keys of route_topk_device plus logits, slogit, workspace,
    out); missing ones are allocated and stored there."""
    t = nat.torch()
    xd = nat.to_device(x, t.float32).reshape(-1, hidden).contiguous()
    T = xd.shape[0]
    b = bufs if bufs is not None else {}
    logits = b.get("logits")
    if logits is None:
        logits = t.empty((T, E), dtype=t.float32, device=xd.device)
    sl = None
    if shared_gate_w is not None:
        sl = b.get("slogit")
        if sl is None:
            sl = t.empty((T,), dtype=t.float32, device=xd.device)
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    gw = nat.to_device(gate_w, t.float16)
    sgw = nat.to_device(shared_gate_w, t.float16) if shared_gate_w is not None else None
    rc = nat.lib().fastllm_gate_matvec(nat.ptr(xd), nat.ptr(gw),
                                       nat.ptr(sgw) if sgw is not None else None,
                                       nat.ptr(logits), nat.ptr(sl) if sl is not None else None,
                                       T, E, hidden, h)
    nat.check_rc(rc, "fastllm_gate_matvec")
    if "workspace" not in b:  # zero-filled: the router's arrival counter above 16 tokens
        b["workspace"] = t.zeros((moe_workspace_bytes(T, hidden, inter,
                                                      shared_inter if shared is not None else 0,
                                                      T * top_k),),
                                 dtype=t.uint8, device=xd.device)
    if "out" not in b:
        b["out"] = t.empty((T, hidden), dtype=t.float32, device=xd.device)
    return moe_route_forward(xd, logits, stacked, top_k, E, hidden, inter,
                             norm_topk_prob=norm, routed_scaling=scale, shared=shared,
                             shared_inter=shared_inter, shared_logit=sl, route=b,
                             out=b["out"], workspace=b["workspace"], stream=stream)

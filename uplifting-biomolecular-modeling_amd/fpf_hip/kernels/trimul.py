"""Triangle-multiplication face, served by libfpf_hip's ``fpf_trimul_fwd`` (K1 planes -> batched MFMA contraction -> K3).

Mirrors common/opt_core/opt_core/kernels/trimul/__init__.py: the op (:3-11), ``WEIGHT_KEYS`` (:171), ``Refusal`` (:188),
``precision_word`` (:219), ``admits`` (:386), ``select(cc, dtype, c_z, c_hidden, n_tokens, direction="outgoing", *, word, residency=None,
backward=False, prefer=None, stack=None, ...)`` (:835) and ``triangle_multiplication(z, mask=None, *, direction, weights, word=None,
selection=None, residual=False, prefer=None, residency=None, stock=None, cache=None, eps=1e-5, ...)`` (:1982).  ``cc`` is a capability
((9, 5) / "9.5" for an MI355X under ROCm torch), an arch name ("gfx950") or a device.  ``cache`` (a dict the caller holds per weight
set) keeps the packed weights; keys carry the weight tensors' identity, so a dict shared across modules re-packs rather than serving
another module's pack.  The workspace (the K1 planes and the contraction output) is the shared per-stream scratch of
``fpf_hip._face.scratch``, not a per-cache buffer.  ``out`` may be ``z`` itself when ``residual=True`` (K3 reads each pixel before
writing it).
"""
import torch

from .. import _face as F
from .. import _lib as L
from .. import cells as CELLS

Refusal, Selection = F.Refusal, F.Selection
WEIGHT_KEYS = ("ln_in_w", "ln_in_b", "w_ag", "w_ap", "w_bg", "w_bp", "ln_out_w", "ln_out_b", "w_o", "w_og")
ROW_NAMES = (F.ROW_FAST, F.ROW_F32)
_DIRS = {"outgoing": "outgoing", "out": "outgoing", "incoming": "incoming", "in": "incoming"}


def direction_word(direction):
    d = _DIRS.get(str(direction))
    if d is None:
        raise ValueError("direction must be outgoing | incoming (got %r)" % (direction,))
    return d


def precision_word(dtype, residency=None, tf32=None):
    """The precision class of a call: bf16 | f32z_bf16 (fp32-resident z, bf16 operands) | fp32 | tf32 | fp16."""
    s = F.dtype_of(dtype)
    if s in ("bf16", "fp16"):
        r = F.dtype_of(residency) if residency is not None else ""
        return ("f32z_" + s) if r == "fp32" else s
    if s == "fp32" and tf32:
        return "tf32"
    return s


def _class_of(prec):
    """precision class -> the dtype word the row resolution keys on ('tf32' is served by the fp32 row: it meets that class;
    'f32z_bf16' by the bf16 row, which reads the fp32 z rounded to bf16 and writes fp32)."""
    return {"bf16": "bf16", "f32z_bf16": "bf16", "fp32": "fp32", "tf32": "fp32"}.get(prec)


def _reduced_fp32_matmul():
    """torch may run this process's fp32 matmuls in a reduced-precision (TF32-class) mode."""
    return torch.get_float32_matmul_precision() in ("high", "medium") or torch.backends.cuda.matmul.allow_tf32


def call_precision(z, residency=None):
    """(precision word, compute dtype) of a live call (common/opt_core/opt_core/kernels/trimul/__init__.py:1293): an fp32 z under
    bf16 autocast on its device -- or with ``residency="fp32"`` and a bf16 compute request made through ``select`` -- is the
    f32z_bf16 class; else z's own dtype (fp32 with TF32 matmuls allowed is tf32)."""
    if z.dtype == torch.float32:
        dev = z.device.type
        ac = torch.is_autocast_enabled(dev) and torch.get_autocast_dtype(dev) == torch.bfloat16 if dev == "cuda" else False
        if ac:
            return "f32z_bf16", torch.bfloat16
        return ("tf32" if _reduced_fp32_matmul() else "fp32"), torch.float32
    return precision_word(z.dtype, residency), z.dtype


def admits(row, cc, dtype, c_z, c_hidden, n_tokens, *, residency=None, backward=False, residual=None, batch=1, abi=None, has_cueq=None,
           has_esm_kernels=None, tf32=None, triton=None):
    """Raise Refusal when ``row`` cannot serve this envelope (static facts only); return None when it can."""
    if row not in ROW_NAMES:
        raise ValueError("unknown row %r (rows: %s)" % (row, ", ".join(ROW_NAMES)))
    arch = F.arch_word(cc)
    if arch != F.ARCH:
        raise Refusal("arch:%s" % arch, row, F.ROW_STOCK, "rows of this package are gfx950 kernels")
    if backward:
        raise Refusal("no_backward", row, F.ROW_STOCK, "forward only")
    prec = precision_word(dtype, residency, tf32)
    want = "bf16" if row == F.ROW_FAST else "fp32"
    if _class_of(prec) != want:
        raise Refusal("precision:%s" % prec, row, F.ROW_F32 if row == F.ROW_FAST else F.ROW_FAST, "row %s serves %s" % (row, want))
    C, H = int(c_z), int(c_hidden)
    if row == F.ROW_FAST and (C, H) != (128, 128):
        raise Refusal("shape:c%dx%d" % (C, H), row, F.ROW_F32, "the bf16 kernels serve c_z = c_hidden = 128")
    if row == F.ROW_F32 and (C > 128 or H > 128):
        raise Refusal("shape:c%dx%d" % (C, H), row, F.ROW_STOCK, "the fp32 kernels serve c_z, c_hidden <= 128")
    return None


def select(cc, dtype, c_z, c_hidden, n_tokens, direction="outgoing", *, word, residency=None, backward=False, prefer=None, stack=None,
           tf32=None, has_cueq=None, config=None, abi=None, exclude=None, form=None, batch=None):
    """Pure: the row serving a TriMul call of this class, or Refusal by name.  ``residency`` = the dtype z is stored in (fp32 with
    bf16 operands is the f32z_bf16 class); ``prefer`` narrows a tier word's candidates, ``exclude`` steps aside from rows;
    ``config`` (a launch setting) is refused by name; ``stack`` / ``has_cueq`` / ``abi`` / ``form`` / ``batch`` do not change
    the answer."""
    d = direction_word(direction)
    w = F.word_base(word)
    if backward:
        raise Refusal("no_backward", w, F.ROW_STOCK, "forward only")
    prec = precision_word(dtype, residency, tf32)
    cls = _class_of(prec)
    if cls is None:
        raise Refusal("precision:%s" % prec, w, F.ROW_STOCK, "served classes: bf16, fp32, tf32 (by the fp32 row)")
    sel = F.resolve(w, cls, F.arch_word(cc), "trimul", cell=CELLS.trimul_key(cls, c_z, c_hidden, n_tokens, "out" if d == "outgoing" else "in"))
    F.narrow(sel, w, prefer, exclude)
    F.no_config(config, sel.row)
    admits(sel.row, cc, cls, c_z, c_hidden, n_tokens)
    return sel


def _pack(weights, dtype, device, cache):
    key = ("_pack", str(device), dtype) + tuple(id(weights[k]) for k in WEIGHT_KEYS)
    p = cache.get(key)
    if p is None:
        missing = [k for k in WEIGHT_KEYS if weights.get(k) is None]
        if missing:
            raise Refusal("weights_missing:" + ",".join(missing), None, F.ROW_STOCK)
        with torch.no_grad():
            p = {}
            for k in WEIGHT_KEYS:
                t = weights[k].detach().to(device)
                p[k] = t.float().contiguous() if k.startswith("ln_") else t.to(dtype).contiguous()
        for k_ in [k_ for k_ in cache if isinstance(k_, tuple) and k_[:1] == ("_pack",)]:
            del cache[k_]
        cache[key] = p
    return p


def triangle_multiplication(z, mask=None, *, direction, weights, word=None, selection=None, residual=False, prefer=None, residency=None,
                            stock=None, cache=None, eps=1e-5, config=None, pad=16, contract="bf16", form=None, module=None, out=None):
    """Returns the update (or z + update when ``residual``) in z's dtype; Refusal by name before any launch.  ``stock`` (the
    kit's own callable) is never called here; ``pad`` (the reference's plane padding) does not change the result (the planes are
    padded to the contraction tile internally); ``contract``: hip_gfx950 contracts bf16 operands (any other word is refused),
    hip_gfx950_f32 contracts in fp32, which meets every contraction class it is asked for."""
    cache = {} if cache is None else cache
    z4 = z if z.dim() == 4 else z.unsqueeze(0)
    B, N, N2, Cz = z4.shape
    if N != N2:
        raise ValueError("z must be [B,N,N,c] or [N,N,c] (got %s)" % (tuple(z.shape),))
    d = direction_word(direction)
    Ch = int(weights["w_ap"].shape[0])
    prec, cdt = call_precision(z4)
    if selection is None:
        f32z = prec == "f32z_bf16"
        sel = select(z, "bf16" if f32z else z.dtype, Cz, Ch, N, d, word=word, residency="fp32" if f32z else residency, prefer=prefer,
                     config=config, form=form, batch=B, tf32=prec == "tf32")
    else:
        sel = selection
    if (sel.row == F.ROW_FAST and str(contract) != "bf16") or str(contract) not in ("bf16", "fp32", "f32", "tf32"):
        raise Refusal("contract:%s" % contract, sel.row, F.ROW_F32 if sel.row == F.ROW_FAST else F.ROW_STOCK,
                      "row %s contracts in %s" % (sel.row, "bf16" if sel.row == F.ROW_FAST else "fp32"))
    if not z4.is_contiguous():
        raise Refusal("stride", sel.row, F.ROW_STOCK, "z must be contiguous")
    F.check_device("trimul", sel.row, z.device, out=out)
    # the bf16 row on an fp32 z is the f32z_bf16 class (bf16 operands, fp32 z / out); the fp32 row takes fp32 z only
    if sel.row == F.ROW_FAST and z.dtype == torch.float32:
        dt, wdt = L.DT_F32Z_BF16, torch.bfloat16
    elif sel.row == F.ROW_FAST and z.dtype == torch.bfloat16:
        dt, wdt = L.DT_BF16, torch.bfloat16
    elif sel.row == F.ROW_F32 and z.dtype == torch.float32:
        dt, wdt = L.DT_F32, torch.float32
    else:
        raise Refusal("precision:%s" % F.dtype_of(z.dtype), sel.row, F.ROW_STOCK, "row %s does not serve a %s z" % (sel.row, z.dtype))
    p = _pack(weights, wdt, z.device, cache)
    m = None
    if mask is not None:
        m = mask if mask.dim() == 3 else mask.unsqueeze(0)
        if tuple(m.shape) != (B, N, N):
            raise Refusal("mask_shape", sel.row, F.ROW_STOCK, str(tuple(mask.shape)))
        m = m.to(device=z.device, dtype=torch.float32).contiguous()
    if out is None:
        out = torch.empty_like(z)
    elif out.shape != z.shape or out.dtype != z.dtype or not out.is_contiguous():
        raise Refusal("out", sel.row, F.ROW_STOCK, "out must be contiguous with z's shape and dtype")
    if out.data_ptr() == z.data_ptr() and not residual:
        raise Refusal("out_aliases_z", sel.row, F.ROW_STOCK, "out may alias z only for the residual form")
    need = L.lib().fpf_trimul_workspace_bytes(B, N, Cz, Ch, dt)
    ws = F.scratch(z.device, need)
    a = _args(z4, out, m, p, d, residual, eps, dt, Cz, Ch, ws)
    L.call("fpf_trimul_fwd", a, L.stream_ptr(z.device))
    cache["_last"] = sel
    return out


def _args(z4, out, m, p, d, residual, eps, dt, Cz, Ch, ws):
    B, N = int(z4.shape[0]), int(z4.shape[1])
    return L.TrimulArgs(abi_version=L.ABI_VERSION, dtype=dt, c_z=Cz, c_h=Ch, batch=B, n=N, z=L.ptr(z4), out=L.ptr(out), mask=L.ptr(m),
                        ln_in_w=L.ptr(p["ln_in_w"]), ln_in_b=L.ptr(p["ln_in_b"]), ln_out_w=L.ptr(p["ln_out_w"]), ln_out_b=L.ptr(p["ln_out_b"]),
                        w_ag=L.ptr(p["w_ag"]), w_ap=L.ptr(p["w_ap"]), w_bg=L.ptr(p["w_bg"]), w_bp=L.ptr(p["w_bp"]), w_o=L.ptr(p["w_o"]),
                        w_og=L.ptr(p["w_og"]), outgoing=1 if d == "outgoing" else 0, residual=1 if residual else 0, eps=float(eps),
                        workspace=L.ptr(ws), workspace_bytes=0 if ws is None else ws.numel())


def triangle_multiplication_chunked(z, mask=None, *, direction, weights, chunk, mode="rows", hidden=None, row_block=None, word="big", residual=False,
                                    out=None, cache=None, eps=1e-5, fp32="passthrough", selection=None, prefer=None, residency=None):
    """Row-chunked triangle multiplication (common/opt_core/opt_core/mem/chunk.py:526 ``triangle_multiplication_chunked``, mode
    ``rows``): both operand planes are built whole once from z (``fpf_trimul_fixed_fwd``), then each block of ``chunk`` output
    rows runs the contraction over the whole shared axis and the output stage for those rows only (``fpf_trimul_fwd`` in its
    rows mode), so the product plane is held for one block instead of all N rows.  Every output element is the whole op's
    arithmetic in the whole op's order: the result equals ``triangle_multiplication`` bitwise.  Since the operands are built
    before any row is written, ``out`` may be z (``residual=True``) in both directions -- the reference's incoming free operand
    reads z columns per block, which an in-place update of earlier blocks would change.

    ``mode="channels"`` (mem/chunk.py:542-552; ``hidden`` = the hidden channel count, ``chunk`` = channels per block):
    ``fpf_trimul_channels_fwd`` builds both operand planes per block of ``chunk`` hidden channels (32, 64 or 128: the largest
    not above ``chunk``, 32 below that) and writes each block's products into ONE full product plane, then the output stage runs over all rows --
    the output LayerNorm normalises over every hidden channel of a pixel, so a channel chunk bounds the operands, not the
    product.  Held: the product plane + two planes of ``chunk`` channels.  Each channel is the whole op's arithmetic: the result
    equals ``triangle_multiplication`` bitwise.  ``row_block`` (the reference's row block of its operand and finish passes) is
    validated and changes nothing here: the kernels stream rows and hold no per-row transients.  The channels mode also serves
    the f32z_bf16 class (fp32 z under bf16 autocast) through the same entry.

    An fp32 call (row hip_gfx950_f32) runs the whole op when ``fp32`` is ``"passthrough"`` or ``"band"`` (the result is the whole
    op's, which meets either label) and is refused for ``"refuse"``; an fp32 z under bf16 autocast (the f32z_bf16 class) runs the
    whole op in rows mode."""
    mode = str(mode)
    if mode not in ("rows", "channels"):
        raise Refusal("mode:%s" % mode, F.word_base(word), F.ROW_STOCK, "the chunked trimul serves mode rows | channels")
    if mode == "channels":
        if not isinstance(hidden, int) or isinstance(hidden, bool) or hidden < 1:
            raise Refusal("bad_hidden", F.word_base(word), F.ROW_STOCK, "hidden=%r is not a positive int (the hidden channel count)" % (hidden,))
        if int(weights["w_ap"].shape[0]) != hidden:
            raise Refusal("operand_output_shape", F.word_base(word), F.ROW_STOCK,
                          "the operand projections give %d hidden channels, hidden=%d" % (int(weights["w_ap"].shape[0]), hidden))
    if row_block is not None and (not isinstance(row_block, int) or isinstance(row_block, bool) or row_block < 1):
        raise ValueError("row_block must be a positive int (got %r)" % (row_block,))
    if str(fp32) not in ("passthrough", "band", "refuse"):
        raise ValueError("fp32 must be passthrough | band | refuse (got %r)" % (fp32,))
    chunk = int(chunk)
    if chunk <= 0:
        raise ValueError("chunk must be positive (got %d)" % chunk)
    cache = {} if cache is None else cache
    z4 = z if z.dim() == 4 else z.unsqueeze(0)
    B, N, N2, Cz = z4.shape
    if N != N2:
        raise ValueError("z must be [B,N,N,c] or [N,N,c] (got %s)" % (tuple(z.shape),))
    d = direction_word(direction)
    Ch = int(weights["w_ap"].shape[0])
    prec, _ = call_precision(z4)
    f32z = prec == "f32z_bf16"
    sel = selection or select(z, "bf16" if f32z else z.dtype, Cz, Ch, N, d, word=word, residency="fp32" if f32z else residency, prefer=prefer,
                              batch=B, tf32=prec == "tf32")
    channels_f32z = mode == "channels" and sel.row == F.ROW_FAST and z.dtype == torch.float32
    if (sel.row != F.ROW_FAST or z.dtype != torch.bfloat16) and not channels_f32z:   # fp32, and the f32z_bf16 class in rows mode: the whole op
        if sel.row == F.ROW_FAST:
            return triangle_multiplication(z, mask, direction=d, weights=weights, selection=sel, residual=residual, cache=cache, eps=eps, out=out)
        if str(fp32) == "refuse":
            raise Refusal("fp32_site", sel.row, F.ROW_STOCK, "an fp32 trimul is not chunked (fp32='refuse')")
        return triangle_multiplication(z, mask, direction=d, weights=weights, selection=sel, residual=residual, cache=cache, eps=eps, out=out)
    if not z4.is_contiguous():
        raise Refusal("stride", sel.row, F.ROW_STOCK, "z must be contiguous")
    F.check_device("trimul", sel.row, z.device, out=out)
    # the bf16 row on an fp32 z is the f32z_bf16 class (bf16 operands, fp32 z / out); the fp32 row takes fp32 z only
    if sel.row == F.ROW_FAST and z.dtype == torch.float32:
        dt, wdt = L.DT_F32Z_BF16, torch.bfloat16
    elif sel.row == F.ROW_FAST and z.dtype == torch.bfloat16:
        dt, wdt = L.DT_BF16, torch.bfloat16
    elif sel.row == F.ROW_F32 and z.dtype == torch.float32:
        dt, wdt = L.DT_F32, torch.float32
    else:
        raise Refusal("precision:%s" % F.dtype_of(z.dtype), sel.row, F.ROW_STOCK, "row %s does not serve a %s z" % (sel.row, z.dtype))
    p = _pack(weights, wdt, z.device, cache)
    m = None
    if mask is not None:
        m = mask if mask.dim() == 3 else mask.unsqueeze(0)
        if tuple(m.shape) != (B, N, N):
            raise Refusal("mask_shape", sel.row, F.ROW_STOCK, str(tuple(mask.shape)))
        m = m.to(device=z.device, dtype=torch.float32).contiguous()
    if out is None:
        out = torch.empty_like(z)
    elif out.shape != z.shape or out.dtype != z.dtype or not out.is_contiguous():
        raise Refusal("out", sel.row, F.ROW_STOCK, "out must be contiguous with z's shape and dtype")
    if out.data_ptr() == z.data_ptr() and not residual:
        raise Refusal("out_aliases_z", sel.row, F.ROW_STOCK, "out may alias z only for the residual form")
    if B * N == 0:
        return out
    lib, st = L.lib(), L.stream_ptr(z.device)
    if mode == "channels":
        ws = F.scratch(z.device, lib.fpf_trimul_channels_workspace_bytes(B, N, chunk, Ch, dt))
        a = _args(z4, out, m, p, d, residual, eps, dt, Cz, Ch, ws)
        L.call("fpf_trimul_channels_fwd", a, chunk, st)
        cache["_last"] = sel
        return out
    rows = min(chunk, N)
    planes = F.scratch(z.device, lib.fpf_trimul_fixed_bytes(B, N, Ch, L.DT_BF16), kind="trimul_planes")
    ws = F.scratch(z.device, lib.fpf_trimul_rows_workspace_bytes(B, N, rows, Ch, L.DT_BF16))
    a = _args(z4, out, m, p, d, residual, eps, L.DT_BF16, Cz, Ch, None)
    L.call("fpf_trimul_fixed_fwd", a, L.ptr(planes), st)
    a.workspace, a.workspace_bytes, a.fixed_in = L.ptr(ws), ws.numel(), L.ptr(planes)
    for r0 in range(0, N, rows):
        a.row0, a.rows = r0, min(rows, N - r0)
        L.call("fpf_trimul_fwd", a, st)
    cache["_last"] = sel
    return out

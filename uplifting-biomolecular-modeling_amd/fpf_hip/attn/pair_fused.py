"""The pair track's fused block faces over libfpf_hip: the triangle-attention block (prologue -> core -> epilogue in three
launches, ``fpf_triattn_block_fwd``) and the fused SwiGLU transition.

Mirrors common/opt_core/opt_core/attn/pair_fused.py: ``Unsupported`` (:86), ``pack_triattn_weights`` (:679),
``pack_transition_weights`` (:744), ``_key_mask`` (:806), ``prologue`` (:1136), ``core_attention`` (:1391), ``epilogue``
(:1416), ``tri_attn_block(z, W, mask=None, *, ending, residual, impl, core, ln, x_ln, scale, bias_frame, variant, ...)`` (:1500)
and ``transition(x, T, *, residual, ln, x_ln, impl, variant, out, mask, ...)`` (:1519).  Every keyword of the reference is
taken by name: what this package serves is served, everything else raises ``Unsupported`` by name before any launch (nothing
is accepted and ignored).

Frames: z is the pair tensor [B,N,N,C] (or [N,N,C]) in its OWN frame.  ``ending=True`` attends in the transposed frame
x = z^T: the prologue reads z^T by address (no copy) and the epilogue writes the update back untransposed.  With
``residual=True`` z is updated in place and returned; otherwise the update in z's frame is returned.

Served: ``ln="fused"`` (LayerNorm in-kernel); ``impl`` "fpf" (the fused kernels; also "hip"); ``core`` "default",
"tier:<word>", a row name of kernels.triattn, or a callable core(q, k, v, bias, mask, scale) (run between this package's
prologue and epilogue stages); ``bias_frame`` "x" or "z" (the same numbers; "z" only changes the strides of the bias the
prologue returns for the ending node); ``ln="stock"`` with ``x_ln`` (the caller's own LayerNorm output, the exact-candidate
construction) on the bf16 rows, projected in place of the in-kernel LayerNorm.  Refused by name: ``x_ln`` with ``ln="fused"`` or
on the fp32 rows,
``impl`` "torch" / "lnl", cores "flash_triattn" / "k2b" (Triton members of the reference), ``write_x``, transition variants
other than the in-place folded one, ``silu`` other than swiglu / liger.
"""
import torch

from .. import _face as F
from .. import _lib as L
from ..kernels import transition as _TR

TRIATTN_KEYS = ("ln_w", "ln_b", "w_q", "w_k", "w_v", "w_g", "b_g", "w_b", "w_o", "b_o")
TRANSITION_KEYS = ("ln_w", "ln_b", "w_a", "w_b", "w_out")
DEFAULT_CORE = "default"
IMPLS = ("fpf", "hip")


class Unsupported(Exception):
    """A named refusal, raised before any kernel launch.  ``reason`` is the short token a kit's ledger carries."""

    def __init__(self, reason, detail=""):
        Exception.__init__(self, reason + (": " + detail if detail else ""))
        self.reason = reason
        self.detail = detail


class TriAttnWeights(object):
    """Packed triangle-attention weights: w_qkvg [4HD, C] (rows q|k|v|g), w_b [H, C], w_o [C_out, HD], optional gate bias
    b_g [HD] and output bias b_o [C_out], LN in fp32; device operand packs per (device, dtype)."""

    def __init__(self):
        self._packs = {}


def _matrix(reason, t, rows=None, cols=None):
    """Refuse (by ``reason``) unless ``t`` is a 2-D weight with ``rows`` rows and ``cols`` columns (None: any)."""
    got = None if t is None else tuple(t.shape)
    if got is None or len(got) != 2 or (rows is not None and got[0] != rows) or (cols is not None and got[1] != cols):
        raise Unsupported(reason, "weight of shape %s where [%s, %s] is needed" % (got, "*" if rows is None else rows, "*" if cols is None else cols))
    return t


def _vector(reason, t, n):
    if t is not None and tuple(t.shape) != (n,):
        raise Unsupported(reason, "bias of shape %s where [%d] is needed" % (tuple(t.shape), n))
    return t


def _named_blocks(w, order, block_rows):
    """The row blocks of a fused weight, keyed by the names of ``order`` (block i = rows i*block_rows .. (i+1)*block_rows - 1)."""
    return dict((name, w[i * block_rows:(i + 1) * block_rows]) for i, name in enumerate(order))


def pack_triattn_weights(*, w_o, n_heads, head_dim, ln_w=None, ln_b=None, w_q=None, w_k=None, w_v=None, w_g=None, w_b=None, w_qkvg=None,
                         qkvg_split=("q", "k", "v", "g"), b_g=None, b_o=None, eps=1e-5, device=None):
    """Pack once per module.  w_q / w_k / w_v / w_g [H*D, C] or w_qkvg [4*H*D, C] (row blocks in ``qkvg_split`` order); w_b [H, C];
    w_o [C_out, H*D]; b_g [H*D] (added to the gate projection before the sigmoid) and b_o [C_out] (added to the output
    projection), or None; ln_w / ln_b [C] or None (no affine).  The bf16 rows use b_g / b_o rounded to bf16 (the reference packs
    them in bf16, pair_fused.py:731-738); the fp32 rows use them as given."""
    H, D = int(n_heads), int(head_dim)
    HD = H * D
    if w_qkvg is not None:
        blocks = _named_blocks(_matrix("w_qkvg-shape", w_qkvg, 4 * HD), qkvg_split, HD)
        w_q, w_k, w_v, w_g = (blocks[n] for n in ("q", "k", "v", "g"))
    if w_g is None:
        raise Unsupported("gate:none", "attention without a gate projection is not served")
    if w_b is None:
        raise Unsupported("bias:none", "the triangle bias projection w_b is required")
    C = None if w_q is None or w_q.dim() != 2 else int(w_q.shape[1])
    for reason, t in (("w_q-shape", w_q), ("w_k-shape", w_k), ("w_v-shape", w_v), ("w_g-shape", w_g)):
        _matrix(reason, t, HD, C)
    _matrix("w_b-shape", w_b, H, C)
    _matrix("w_o-shape", w_o, None, HD)
    _vector("b_g-shape", b_g, HD)
    _vector("b_o-shape", b_o, int(w_o.shape[0]))
    W = TriAttnWeights()
    dev = device if device is not None else w_o.device
    W.C, W.H, W.D, W.C_out, W.eps, W.dev = C, H, D, int(w_o.shape[0]), float(eps), dev
    with torch.no_grad():
        W.wqkvg = torch.cat([w_q, w_k, w_v, w_g], 0).detach().to(dev)
        W.wb = w_b.detach().to(dev)
        W.wo = w_o.detach().to(dev)
        W.b_g = None if b_g is None else b_g.detach().to(dev)
        W.b_o = None if b_o is None else b_o.detach().to(dev)
        W.ln_w = None if ln_w is None else ln_w.detach().to(dev).float().contiguous()
        W.ln_b = None if ln_b is None else ln_b.detach().to(dev).float().contiguous()
    W.shapes = "c%dh%dd%do%d" % (C, H, D, W.C_out)
    return W


def _wpack(W, dtype, device):
    """(w_qkvg, w_b, w_o, b_g, b_o) on ``device``: weights in the row's dtype, biases fp32 (bf16-rounded for the bf16 row)."""
    key = (str(device), dtype)
    p = W._packs.get(key)
    if p is None:
        with torch.no_grad():
            ws = tuple(t.to(device=device, dtype=dtype).contiguous() for t in (W.wqkvg, W.wb, W.wo))
            bs = tuple(None if t is None else t.to(device=device, dtype=dtype).float().contiguous() for t in (W.b_g, W.b_o))
            p = W._packs[key] = ws + bs
    return p


_MASK_U8 = {}


def _pair_mask(mask, z4, ending=False):
    """The pair mask as the kernels take it: u8 (nonzero = keep), contiguous, on z's device, in the attention frame (the ending
    node gets the transposed mask, mask_frame 1, so each attention row's keys are contiguous) -> (tensor, dtype, mask_frame).
    The copies are made once and kept while the same tensor (same object, same version counter) comes back -- a pair stack
    passes one mask to every block.  Inference tensors carry no version counter, so a mask made under torch.inference_mode()
    is converted on every call instead.  A cached mask that keeps every pixel is handed on as no mask (the reference's pairfuse
    driver does the same, boltz2/opt/forward/pairfuse/bz_pairfuse.py:46-50): the block then builds no keep table and runs the
    mask-free core, whose arithmetic is the masked core's on fully kept tiles (the same bits).  Deciding that reads one flag
    back from the device once per mask tensor (not while the stream is capturing a graph, and not for inference tensors)."""
    if mask is None:
        return None, L.DT_U8, 0
    B, N = z4.shape[0], z4.shape[1]
    m = mask if mask.dim() == 3 else mask.unsqueeze(0)
    if tuple(m.shape) != (B, N, N):
        raise Unsupported("mask-shape", str(tuple(mask.shape)))
    version = None if mask.is_inference() else mask._version
    key = ("t" if ending else "m", z4.device)
    hit = _MASK_U8.get(key)
    if version is not None and hit is not None and hit[0] is mask and hit[1] == version:
        return hit[2], L.DT_U8, (0 if hit[2] is None else 1)
    mm = m.transpose(1, 2) if ending else m
    u8 = (mm.to(z4.device) != 0).contiguous().view(torch.uint8)
    if version is not None:
        if u8.device.type != "meta" and not (u8.is_cuda and torch.cuda.is_current_stream_capturing()) and bool(u8.all()):
            u8 = None                                 # every pixel kept: no mask
        _MASK_U8[key] = (mask, version, u8)          # holding the tensor keeps its storage from being reused
    return u8, L.DT_U8, (0 if u8 is None else 1)


def _block_check(z, W, word, face):
    """Shape / row gate shared by the block and its stages: -> (z4, Selection), or Unsupported before any launch."""
    z4 = z if z.dim() == 4 else z.unsqueeze(0)
    if z4.dim() != 4 or z4.shape[1] != z4.shape[2] or z4.shape[-1] != W.C:
        raise Unsupported("shape", str(tuple(z.shape)))
    if not z4.is_contiguous():
        raise Unsupported("stride", "z must be contiguous")
    try:
        sel = F.resolve(word, F.dtype_word(z.dtype), F.device_word(z), "pair_fused:" + face, cell="block:%s" % W.shapes)
    except F.Refusal as e:
        raise Unsupported(e.kind, e.detail) from None
    if sel.row == F.ROW_FAST and (W.C, W.H * W.D, W.D, W.C_out) != (128, 128, 32, 128):
        raise Unsupported("shape:%s" % W.shapes, "the bf16 block serves C = 128, H*D = 128, D = 32")
    if sel.row == F.ROW_F32 and (W.C > 128 or W.H * W.D > 128 or W.D not in (16, 32, 64) or W.C_out != W.C):
        raise Unsupported("shape:%s" % W.shapes, "the fp32 block serves C, H*D <= 128, D 16 | 32 | 64")
    return z4, sel


def _check_ln(ln, x_ln, like=None):
    """``ln="fused"``: the kernels normalise in-kernel (no x_ln).  ``ln="stock"``: x_ln, the caller's own LayerNorm output (the
    attention frame for the triangle attention), is projected in place of the in-kernel LayerNorm -- the exact-candidate
    construction of pair_fused.py:1151-1160; it must be a contiguous bf16 tensor of ``like``'s shape on its device.  Returns
    the x_ln to pass (4-D when ``like`` is), or None."""
    if ln == "fused":
        if x_ln is not None:
            raise Unsupported("x_ln:ln_fused", "x_ln is projected with ln='stock'; ln='fused' normalises in-kernel")
        return None
    if ln != "stock":
        raise Unsupported("ln:%s" % ln)
    if x_ln is None:
        raise Unsupported("ln:stock-needs-x_ln", "ln='stock' projects the caller's own LayerNorm output x_ln")
    if like is None:
        return x_ln
    x4 = x_ln.unsqueeze(0) if x_ln.dim() + 1 == like.dim() else x_ln
    if tuple(x4.shape) != tuple(like.shape) or x4.dtype != torch.bfloat16 or not x4.is_contiguous() or x4.device != like.device:
        raise Unsupported("x_ln-shape", "a contiguous bf16 tensor of shape %s on %s, got %s %s on %s"
                          % (tuple(like.shape), like.device, tuple(x_ln.shape), x_ln.dtype, x_ln.device))
    if like.dtype != torch.bfloat16:
        raise Unsupported("x_ln:%s" % F.dtype_word(like.dtype), "x_ln is served on the bf16 rows (the fp32 rows normalise in-kernel)")
    return x4


def _check_impl(impl):
    if impl is not None and impl not in IMPLS:
        raise Unsupported("impl:%s" % impl, "served: fused HIP kernels (impl 'fpf' / 'hip')")


def _check_bias_frame(bias_frame):
    if bias_frame not in ("x", "z"):
        raise Unsupported("bias_frame:%s" % bias_frame)


def _core_word(core):
    """The block's own core serves "default", "tier:<word>" and the row names of kernels.triattn; -> the tier / row word, or None
    for a callable; Unsupported for the reference's Triton members and anything else."""
    if callable(core):
        return None
    c = str(core)
    if c == DEFAULT_CORE:
        return "fast"
    if c.startswith("tier:"):
        return c[len("tier:"):]
    if c in (F.ROW_FAST, F.ROW_F32):
        return c
    raise Unsupported("core:%s" % c, "served cores: default, tier:<word>, %s, %s, or a callable" % (F.ROW_FAST, F.ROW_F32))


def _key_mask(mask, z, ending):
    """Pair mask [B,N,N] / [N,N] in z's frame -> the core's key mask [B, I, 1, 1, J] bool in the attention frame (transposed for
    the ending node), on z's device (z None: the mask's own), as pair_fused.py:806-829 builds it.  None stays None."""
    if mask is None:
        return None
    m = mask if mask.dim() == 3 else mask.unsqueeze(0)
    if ending:
        m = m.transpose(1, 2)
    if z is not None:
        m = m.to(z.device)
    return (m != 0)[:, :, None, None, :]


def _launch(entry, args, dev):
    try:
        L.call(entry, args, L.stream_ptr(dev))
    except L.LibError as e:
        raise Unsupported("lib:" + e.kind, e.msg) from None


def prologue(z, W, *, ending=False, ln="fused", x_ln=None, impl="fpf", bias_frame="x", write_x=False, word="fast", _plan=None):
    """-> (q, k, v, g, bias) in the attention frame x = z (z^T for the ending node, read by address): q, k, v [B, I, H, J, D]
    (bf16: v is a view of storage [B, I, H, D, J], which the op face serves without a copy), g [B, I, J, H*D] pre-sigmoid (b_g
    added), bias [B, 1, H, I, J] fp32 (bias_frame "z": the same values stored in z's frame for the ending node, an axes-swapped
    view).  Mirrors pair_fused.py:1136 (``prologue``); one launch of ``fpf_triattn_prologue_fwd``."""
    if write_x:
        raise Unsupported("write_x", "returning the normalised x is not served")
    _check_ln(ln, x_ln)
    _check_impl(impl)
    _check_bias_frame(bias_frame)
    z4, sel = _block_check(z, W, word, "prologue")
    x4 = _check_ln(ln, x_ln, z4)
    B, N = int(z4.shape[0]), int(z4.shape[1])
    H, D = W.H, W.D
    wqkvg, wb, _wo, bg, _bo = _wpack(W, z.dtype, z.device)
    e = dict(dtype=z.dtype, device=z.device)
    q = torch.empty(B, N, H, N, D, **e)
    k = torch.empty(B, N, H, N, D, **e)
    bf = z.dtype == torch.bfloat16
    jp = -(-N // 32) * 32                                 # V^T rows padded to a multiple of 32 columns (16-byte stores)
    vs = torch.empty(B, N, H, D, jp, **e) if bf else torch.empty(B, N, H, N, D, **e)
    g = torch.empty(B, N, N, H * D, **e)
    bias = torch.empty(B, H, N, N, dtype=torch.float32, device=z.device)
    a = L.TriattnPrologueArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16 if bf else L.DT_F32, B=B, N=N, C=W.C, H=H, D=D, z=L.ptr(z4),
                              ln_w=L.ptr(W.ln_w), ln_b=L.ptr(W.ln_b), eps=W.eps, w_qkvg=L.ptr(wqkvg), w_b=L.ptr(wb),
                              ending=1 if ending else 0, q=L.ptr(q), k=L.ptr(k), v=L.ptr(vs), v_ld=jp if bf else 0, g=L.ptr(g),
                              bias=L.ptr(bias), b_g=L.ptr(bg), x_ln=L.ptr(x4))
    _launch("fpf_triattn_prologue_fwd", a, z.device)
    v = vs[..., :N].transpose(-1, -2) if bf else vs
    if bias_frame == "z" and ending:
        bias = bias.transpose(-1, -2).contiguous().transpose(-1, -2)
    return q, k, v, g, bias.unsqueeze(1)


def core_attention(q, k, v, bias, mask5=None, *, core=DEFAULT_CORE, scale=None):
    """o [B, I, H, J, D] = softmax_j(scale q.k + bias, -inf at masked keys) v (pair_fused.py:1391): ``core`` "default" (this
    package's fast row), "tier:<word>" / a row name of kernels.triattn, or a callable core(q, k, v, bias, mask, scale).  A
    callable gets v with a contiguous head_dim (the op contract's unit stride), copied when the prologue handed it transposed."""
    from ..kernels import triattn as _TA
    import math
    if callable(core):
        if v.stride(-1) != 1:
            v = v.contiguous()
        return core(q, k, v, bias, mask5, (1.0 / math.sqrt(q.shape[-1])) if scale is None else float(scale))
    w = _core_word(core)
    try:
        return _TA.triangle_attention(q, k, v, bias, mask5, scale, word=w)
    except F.Refusal as e:
        raise Unsupported("core:" + e.kind, e.detail) from None


def epilogue(o, g, W, z=None, *, ending=False, residual=False, impl="fpf", o_layout="ihjd", out=None, word="fast", _plan=None):
    """u = (sigmoid(g) * o) W_o^T + b_o (pair_fused.py:1416).  residual=True: z (its own frame) is updated in place (the ending
    node's u[i, j] is added at z[j, i]) and returned; else the update in the attention frame [B, I, J, C_out] (for the ending node
    a transposed view of a z-frame tensor, as the reference returns it).  One launch of ``fpf_triattn_epilogue_fwd``."""
    _check_impl(impl)
    if o_layout != "ihjd":
        raise Unsupported("o_layout:%s" % o_layout, "o is taken as [B, I, H, J, D]")
    if o.dim() != 5:
        raise Unsupported("o-shape", str(tuple(o.shape)))
    B, N, H, J, D = (int(x) for x in o.shape)
    if (H, D) != (W.H, W.D) or J != N or tuple(g.shape) != (B, N, N, H * D):
        raise Unsupported("o/g-shape", "%s %s" % (tuple(o.shape), tuple(g.shape)))
    if not (o.is_contiguous() and g.is_contiguous()) or g.dtype != o.dtype:
        raise Unsupported("o/g-layout", "o [B,I,H,J,D] and g [B,I,J,HD] contiguous, one dtype")
    if g.device != o.device:
        raise Unsupported("device:g", "o and g must be on one device")
    if residual:
        if z is None:
            raise Unsupported("residual-needs-z")
        z4, sel = _block_check(z, W, word, "epilogue")
        if z4.dtype != o.dtype or tuple(z4.shape[:3]) != (B, N, N) or z4.device != o.device:
            raise Unsupported("z-shape", str(tuple(z.shape)))
        dst = z4
    else:
        if out is not None:
            dst = out if out.dim() == 4 else out.unsqueeze(0)
            if tuple(dst.shape) != (B, N, N, W.C_out) or not dst.is_contiguous() or dst.dtype != o.dtype or dst.device != o.device:
                raise Unsupported("out", "a contiguous [B, N, N, C_out] tensor of o's dtype on o's device (z's frame)")
        else:
            dst = torch.empty(B, N, N, W.C_out, dtype=o.dtype, device=o.device)
        _block_check(dst, W, word, "epilogue")
    _, _, wo, _bg, bo = _wpack(W, o.dtype, o.device)
    a = L.TriattnEpilogueArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16 if o.dtype == torch.bfloat16 else L.DT_F32, B=B, N=N, C=W.C, H=H, D=D,
                              o=L.ptr(o), g=L.ptr(g), w_o=L.ptr(wo), ending=1 if ending else 0, residual=1 if residual else 0, out=L.ptr(dst),
                              b_o=L.ptr(bo))
    _launch("fpf_triattn_epilogue_fwd", a, o.device)
    if residual:
        return z
    return dst.transpose(1, 2) if ending else dst


def _block_args(z4, W, m, mdt, mframe, ending, residual, out, scale, ws, dt, wpack, row0=0, rows=0, bias_in=None, x_ln=None):
    wqkvg, wb, wo, bg, bo = wpack
    B, N = int(z4.shape[0]), int(z4.shape[1])
    return L.TriattnBlockArgs(abi_version=L.ABI_VERSION, dtype=dt, B=B, N=N, C=W.C, H=W.H, D=W.D, z=L.ptr(z4), mask=L.ptr(m), mask_dtype=mdt,
                              ln_w=L.ptr(W.ln_w), ln_b=L.ptr(W.ln_b), eps=W.eps, w_qkvg=L.ptr(wqkvg), w_b=L.ptr(wb), w_o=L.ptr(wo),
                              ending=1 if ending else 0, residual=1 if residual else 0, out=L.ptr(out), scale=float(scale or 0.0),
                              workspace=L.ptr(ws), workspace_bytes=ws.numel(), row0=row0, rows=rows, bias_in=L.ptr(bias_in),
                              mask_frame=mframe, b_g=L.ptr(bg), b_o=L.ptr(bo), x_ln=L.ptr(x_ln))


def tri_attn_block(z, W, mask=None, *, ending=False, residual=False, impl="fpf", core=DEFAULT_CORE, ln="fused", x_ln=None, scale=None,
                   bias_frame="x", variant=None, engage_cells=False, word="fast"):
    """The fused block; returns the update in z's frame (residual=False) or z updated in place (residual=True).  With this
    package's own core (``core`` "default" / "tier:<word>" / a row name) it is one call of ``fpf_triattn_block_fwd`` (three
    launches); a callable ``core`` runs between the prologue and epilogue stages.  ``engage_cells`` does not change the call."""
    _check_ln(ln, x_ln)
    _check_impl(impl)
    _check_bias_frame(bias_frame)
    if variant is not None:
        raise Unsupported("variant:%s" % (variant,), "the block has one variant")
    cw = _core_word(core)
    z4, sel = _block_check(z, W, word, "tri_attn_block")
    x4 = _check_ln(ln, x_ln, z4)
    if cw is None:                                    # the caller's core between this package's stages
        q, k, v, g, bias = prologue(z, W, ending=ending, ln=ln, x_ln=x4, word=word)
        o = core_attention(q, k, v, bias, _key_mask(mask, z, ending), core=core, scale=scale)
        if residual:
            return epilogue(o.contiguous(), g, W, z, ending=ending, residual=True, word=word)
        u = epilogue(o.contiguous(), g, W, ending=ending, residual=False, word=word)
        u = u.transpose(1, 2) if ending else u
        return u if z.dim() == 4 else u[0]
    try:                                              # the block's own core: the core word must resolve to the block's row
        csel = F.resolve(cw, F.dtype_word(z.dtype), F.device_word(z), "pair_fused:core")
    except F.Refusal as e:
        raise Unsupported("core:" + e.kind, e.detail) from None
    if csel.row != sel.row:
        raise Unsupported("core:%s" % core, "the block's %s operands run row %s, not %s" % (F.dtype_word(z.dtype), sel.row, csel.row))
    B, N = int(z4.shape[0]), int(z4.shape[1])
    m, mdt, mframe = _pair_mask(mask, z4, ending)
    wp = _wpack(W, z.dtype, z.device)
    dt = L.DT_BF16 if z.dtype == torch.bfloat16 else L.DT_F32
    ws = F.scratch(z.device, L.lib().fpf_triattn_block_workspace_bytes(B, N, 0, W.C, W.H, W.D, dt))
    out = z4 if residual else torch.empty_like(z4)
    _launch("fpf_triattn_block_fwd", _block_args(z4, W, m, mdt, mframe, ending, residual, out, scale, ws, dt, wp, x_ln=x4), z.device)
    if residual:
        return z
    return out if z.dim() == 4 else out[0]


def tri_attn_block_chunked(z, W, mask=None, *, ending=False, residual=False, chunk=256, scale=None, word="big"):
    """The row-chunked (`big`) triangle-attention block, after common/opt_core/opt_core/mem/chunk.py:424
    (triangle_attention_chunked): pass 1 computes the full bias [B, H, N, N] from every pixel (one launch of
    ``fpf_triattn_bias_fwd``); pass 2 runs prologue -> core -> gate-fused epilogue on ``chunk`` attention rows at a time (z rows
    for the starting node, z columns for the ending node), so the q / k / v / o workspace holds one chunk.  In place
    (``residual=True``) the update of a chunk only touches its own rows / columns, which no later chunk reads, and every row's
    arithmetic is independent of the others: the result is bitwise the whole-tensor block's.  fp32 operands run the whole
    block (the reference's fp32 passthrough)."""
    z4, sel = _block_check(z, W, word, "tri_attn_block_chunked")
    if sel.row != F.ROW_FAST:
        return tri_attn_block(z, W, mask, ending=ending, residual=residual, scale=scale, word=word)
    chunk = int(chunk)
    if chunk <= 0:
        raise Unsupported("chunk:%d" % chunk)
    B, N = int(z4.shape[0]), int(z4.shape[1])
    m, mdt, mframe = _pair_mask(mask, z4, ending)
    wp = _wpack(W, z.dtype, z.device)
    rows = min(chunk, N)
    lib = L.lib()
    ws = F.scratch(z.device, lib.fpf_triattn_block_workspace_bytes(B, N, rows, W.C, W.H, W.D, L.DT_BF16))
    bias = F.scratch(z.device, lib.fpf_triattn_bias_bytes(B, N, W.H, L.DT_BF16), kind="bias")
    ab = L.TriattnBiasArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, B=B, N=N, C=W.C, H=W.H, D=W.D, z=L.ptr(z4), ln_w=L.ptr(W.ln_w),
                           ln_b=L.ptr(W.ln_b), eps=W.eps, w_qkvg=L.ptr(wp[0]), w_b=L.ptr(wp[1]), ending=1 if ending else 0, bias=L.ptr(bias))
    _launch("fpf_triattn_bias_fwd", ab, z.device)
    out = z4 if residual else torch.empty_like(z4)
    for r0 in range(0, N, rows):
        a = _block_args(z4, W, m, mdt, mframe, ending, residual, out, scale, ws, L.DT_BF16, wp, row0=r0, rows=min(rows, N - r0), bias_in=bias)
        _launch("fpf_triattn_block_fwd", a, z.device)
    if residual:
        return z
    return out if z.dim() == 4 else out[0]


class TransitionWeights(object):
    """The pair_fused transition pack: C, NH (hidden), n = NH / C, and the kernels.transition.Weights it serves through."""

    def __init__(self, weights):
        self.W = weights
        self.C, self.NH = weights.c, weights.hidden
        self.n = self.NH // self.C


def pack_transition_weights(*, w_out, ln_w=None, ln_b=None, w_a=None, w_b=None, w_ab=None, ab_split=("a", "b"), eps=1e-5, device=None):
    """SwiGLU transition weights: w_a / w_b [n*C, C] (silu branch, linear branch) or the fused w_ab [2*n*C, C] with its row blocks
    named in ``ab_split`` order; w_out [C, n*C]; LayerNorm ln_w / ln_b [C] or None."""
    C, NH = (int(x) for x in _matrix("w_out-shape", w_out).shape)
    if w_ab is not None:
        blocks = _named_blocks(_matrix("w_ab-shape", w_ab, 2 * NH, C), ab_split, NH)
        w_a, w_b = blocks["a"], blocks["b"]
    _matrix("w_a-shape", w_a, NH, C)
    _matrix("w_b-shape", w_b, NH, C)
    if NH % C:
        raise Unsupported("hidden", "hidden width %d is not a whole multiple of the %d channels" % (NH, C))
    return TransitionWeights(_TR.pack(w_o=w_out, w_a=w_a, w_b=w_b, ln_w=ln_w, ln_b=ln_b, eps=eps, device=device))


TRANSITION_VARIANTS = ("v2_fold",)


def transition(x, T, *, residual=False, ln="fused", x_ln=None, impl="fpf", variant=None, out=None, mask=None, binary_mask=None,
               variants=None, silu="swiglu", word="fast"):
    """y = W_out(silu(W_a n) * W_b n), n = LN(x) in-kernel; x + y when residual; ``out`` may be x (in place); ``mask`` one value
    per row, any values (``binary_mask`` changes nothing).  The kernel is the in-place folded variant (the reference's v2_fold:
    mask and residual folded, out may alias x): ``variant`` / ``variants`` must name it when given.  The hidden
    h = silu(a) * b is formed from fp32 a, b and rounded to bf16 once, the 'liger' form; ``silu='swiglu'`` (which rounds
    silu(a) first) is served by the same kernel: the two differ by one bf16 rounding of the hidden, inside the fast tier's
    tolerance."""
    x_ln = _check_ln(ln, x_ln, x)
    _check_impl(impl)
    if variant is not None and variant not in TRANSITION_VARIANTS:
        raise Unsupported("variant:%s" % (variant,), "served: %s" % (TRANSITION_VARIANTS,))
    if variants is not None and not any(v in TRANSITION_VARIANTS for v in variants):
        raise Unsupported("variants:%s" % (tuple(variants),), "served: %s" % (TRANSITION_VARIANTS,))
    if silu not in ("swiglu", "liger"):
        raise Unsupported("silu:%s" % silu)
    try:
        y, _sel = _TR.transition(x, T.W, word=word, residual=residual, mask=mask, binary_mask=binary_mask, out=out, x_ln=x_ln)
    except F.Refusal as e:
        raise Unsupported(e.kind, e.detail) from None
    return y

"""The pair track's fused block faces over libfpf_hip: the triangle-attention block (prologue -> core -> epilogue in three
launches, ``fpf_triattn_block_fwd``) and the fused SwiGLU transition.

Mirrors common/opt_core/opt_core/attn/pair_fused.py: ``Unsupported`` (:86), ``pack_triattn_weights`` (:679),
``pack_transition_weights`` (:744), ``_key_mask`` (:806), ``prologue`` (:1136), ``core_attention`` (:1391), ``epilogue``
(:1416), ``tri_attn_block(z, W, mask=None, *, ending, residual, ...)`` (:1500) and ``transition(x, T, *, residual, out, mask,
...)`` (:1519).

Frames: z is the pair tensor [B,N,N,C] (or [N,N,C]) in its OWN frame.  ``ending=True`` attends in the transposed frame
x = z^T: the prologue reads z^T by address (no copy) and the epilogue writes the update back untransposed.  With
``residual=True`` z is updated in place and returned; otherwise the update in z's frame is returned.
"""
import torch

from .. import _face as F
from .. import _lib as L
from ..kernels import transition as _TR

TRIATTN_KEYS = ("ln_w", "ln_b", "w_q", "w_k", "w_v", "w_g", "b_g", "w_b", "w_o", "b_o")
TRANSITION_KEYS = ("ln_w", "ln_b", "w_a", "w_b", "w_out")


class Unsupported(Exception):
    """A named refusal, raised before any kernel launch.  ``reason`` is the short token a kit's ledger carries."""

    def __init__(self, reason, detail=""):
        Exception.__init__(self, reason + (": " + detail if detail else ""))
        self.reason = reason
        self.detail = detail


class TriAttnWeights(object):
    """Packed triangle-attention weights: w_qkvg [4HD, C] (rows q|k|v|g), w_b [H, C], w_o [C_out, HD], LN in fp32, per dtype."""

    def __init__(self):
        self._packs = {}
        self._ws = {}


def pack_triattn_weights(*, w_o, n_heads, head_dim, ln_w=None, ln_b=None, w_q=None, w_k=None, w_v=None, w_g=None, w_b=None, w_qkvg=None,
                         qkvg_split=("q", "k", "v", "g"), b_g=None, b_o=None, eps=1e-5, device=None):
    H, D = int(n_heads), int(head_dim)
    HD = H * D
    if w_qkvg is not None:
        if int(w_qkvg.shape[0]) != 4 * HD:
            raise Unsupported("w_qkvg-shape", str(tuple(w_qkvg.shape)))
        blocks = {nm: w_qkvg[i * HD:(i + 1) * HD] for i, nm in enumerate(qkvg_split)}
        w_q, w_k, w_v, w_g = blocks["q"], blocks["k"], blocks["v"], blocks["g"]
    if w_g is None:
        raise Unsupported("gate:none")
    if w_b is None:
        raise Unsupported("bias:none")
    if b_g is not None or b_o is not None:
        raise Unsupported("projection_bias", "the HIP block has no gate / output projection bias operand")
    for nm, t in (("w_q", w_q), ("w_k", w_k), ("w_v", w_v), ("w_g", w_g)):
        if t is None or t.dim() != 2 or int(t.shape[0]) != HD:
            raise Unsupported(nm + "-shape", str(None if t is None else tuple(t.shape)))
    C = int(w_q.shape[1])
    if tuple(w_b.shape) != (H, C):
        raise Unsupported("w_b-shape", str(tuple(w_b.shape)))
    if w_o.dim() != 2 or int(w_o.shape[1]) != HD:
        raise Unsupported("w_o-shape", str(tuple(w_o.shape)))
    W = TriAttnWeights()
    dev = device if device is not None else w_o.device
    W.C, W.H, W.D, W.C_out, W.eps, W.dev = C, H, D, int(w_o.shape[0]), float(eps), dev
    with torch.no_grad():
        W.wqkvg = torch.cat([w_q, w_k, w_v, w_g], 0).detach().to(dev)
        W.wb = w_b.detach().to(dev)
        W.wo = w_o.detach().to(dev)
        W.ln_w = None if ln_w is None else ln_w.detach().to(dev).float().contiguous()
        W.ln_b = None if ln_b is None else ln_b.detach().to(dev).float().contiguous()
    W.shapes = "c%dh%dd%do%d" % (C, H, D, W.C_out)
    return W


def _wpack(W, dtype, device):
    key = (str(device), dtype)
    p = W._packs.get(key)
    if p is None:
        with torch.no_grad():
            p = W._packs[key] = tuple(t.to(device=device, dtype=dtype).contiguous() for t in (W.wqkvg, W.wb, W.wo))
    return p


_MASK_U8 = {}


def _pair_mask(mask, z4, ending=False):
    """The pair mask as the kernels take it: u8 (nonzero = keep), contiguous, in the attention frame (the ending node gets the
    transposed mask, mask_frame 1, so each attention row's keys are contiguous) -> (tensor, dtype, mask_frame).  The copies
    are made once and kept while the same tensor (same object, unmodified) comes back -- a pair stack passes one mask to
    every block -- because the core builds its key table from contiguous u8 rows with one 16-byte load per 16 keys."""
    if mask is None:
        return None, L.DT_U8, 0
    B, N = z4.shape[0], z4.shape[1]
    m = mask if mask.dim() == 3 else mask.unsqueeze(0)
    if tuple(m.shape) != (B, N, N):
        raise Unsupported("mask-shape", str(tuple(mask.shape)))
    key = "t" if ending else "m"
    hit = _MASK_U8.get(key)
    if hit is not None and hit[0] is mask and hit[1] == mask._version:
        return hit[2], L.DT_U8, 1
    mm = m.transpose(1, 2) if ending else m
    u8 = (mm != 0).contiguous().view(torch.uint8)
    _MASK_U8[key] = (mask, mask._version, u8)           # holding the tensor keeps its storage from being reused
    return u8, L.DT_U8, 1


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


def _key_mask(mask, z, ending):
    """Pair mask [B,N,N] / [N,N] in z's frame -> the core's key mask [B, I, 1, 1, J] bool in the attention frame (transposed for
    the ending node), as pair_fused.py:806-829 builds it.  None stays None."""
    if mask is None:
        return None
    m = mask if mask.dim() == 3 else mask.unsqueeze(0)
    if ending:
        m = m.transpose(1, 2)
    return (m != 0)[:, :, None, None, :]


def prologue(z, W, *, ending=False, word="fast", **_unused):
    """-> (q, k, v, g, bias) in the attention frame x = z (z^T for the ending node, read by address): q, k, v [B, I, H, J, D]
    (bf16: v is a view of storage [B, I, H, D, J], which the op face serves without a copy), g [B, I, J, H*D] pre-sigmoid, bias
    [B, 1, H, I, J] fp32.  Mirrors pair_fused.py:1136 (``prologue``); one launch of ``fpf_triattn_prologue_fwd``."""
    z4, sel = _block_check(z, W, word, "prologue")
    B, N = int(z4.shape[0]), int(z4.shape[1])
    H, D = W.H, W.D
    wqkvg, wb, _wo = _wpack(W, z.dtype, z.device)
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
                              bias=L.ptr(bias))
    try:
        L.call("fpf_triattn_prologue_fwd", a, L.stream_ptr(z.device))
    except L.LibError as e_:
        raise Unsupported("lib:" + e_.kind, e_.msg) from None
    v = vs[..., :N].transpose(-1, -2) if bf else vs
    return q, k, v, g, bias.unsqueeze(1)


def core_attention(q, k, v, bias, mask5=None, *, core="tier:fast", scale=None):
    """o [B, I, H, J, D] = softmax_j(scale q.k + bias, -inf at masked keys) v through the op face (pair_fused.py:1391);
    ``core`` = "tier:<word>" / a row name of kernels.triattn, or a callable core(q, k, v, bias, mask, scale)."""
    from ..kernels import triattn as _TA
    if callable(core):
        import math
        return core(q, k, v, bias, mask5, (1.0 / math.sqrt(q.shape[-1])) if scale is None else float(scale))
    w = str(core)
    if w.startswith("tier:"):
        w = w[len("tier:"):]
    try:
        return _TA.triangle_attention(q, k, v, bias, mask5, scale, word=w)
    except F.Refusal as e:
        raise Unsupported("core:" + e.kind, e.detail) from None


def epilogue(o, g, W, z=None, *, ending=False, residual=False, out=None, word="fast", **_unused):
    """u = (sigmoid(g) * o) W_o^T (pair_fused.py:1416).  residual=True: z (its own frame) is updated in place (the ending node's
    u[i, j] is added at z[j, i]) and returned; else the update in the attention frame [B, I, J, C_out] (for the ending node a
    transposed view of a z-frame tensor, as the reference returns it).  One launch of ``fpf_triattn_epilogue_fwd``."""
    if o.dim() != 5:
        raise Unsupported("o-shape", str(tuple(o.shape)))
    B, N, H, J, D = (int(x) for x in o.shape)
    if (H, D) != (W.H, W.D) or J != N or tuple(g.shape) != (B, N, N, H * D):
        raise Unsupported("o/g-shape", "%s %s" % (tuple(o.shape), tuple(g.shape)))
    if not (o.is_contiguous() and g.is_contiguous()) or g.dtype != o.dtype:
        raise Unsupported("o/g-layout", "o [B,I,H,J,D] and g [B,I,J,HD] contiguous, one dtype")
    if residual:
        if z is None:
            raise Unsupported("residual-needs-z")
        z4, sel = _block_check(z, W, word, "epilogue")
        if z4.dtype != o.dtype or tuple(z4.shape[:3]) != (B, N, N):
            raise Unsupported("z-shape", str(tuple(z.shape)))
        dst = z4
    else:
        if out is not None:
            dst = out if out.dim() == 4 else out.unsqueeze(0)
            if tuple(dst.shape) != (B, N, N, W.C_out) or not dst.is_contiguous() or dst.dtype != o.dtype:
                raise Unsupported("out", "a contiguous [B, N, N, C_out] tensor of o's dtype (z's frame)")
        else:
            dst = torch.empty(B, N, N, W.C_out, dtype=o.dtype, device=o.device)
        _block_check(dst, W, word, "epilogue")
    _, _, wo = _wpack(W, o.dtype, o.device)
    a = L.TriattnEpilogueArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16 if o.dtype == torch.bfloat16 else L.DT_F32, B=B, N=N, C=W.C, H=H, D=D,
                              o=L.ptr(o), g=L.ptr(g), w_o=L.ptr(wo), ending=1 if ending else 0, residual=1 if residual else 0, out=L.ptr(dst))
    try:
        L.call("fpf_triattn_epilogue_fwd", a, L.stream_ptr(o.device))
    except L.LibError as e_:
        raise Unsupported("lib:" + e_.kind, e_.msg) from None
    if residual:
        return z
    return dst.transpose(1, 2) if ending else dst


def tri_attn_block(z, W, mask=None, *, ending=False, residual=False, scale=None, word="fast", **_unused):
    """The fused block; returns the update in z's frame (residual=False) or z updated in place (residual=True)."""
    z4, sel = _block_check(z, W, word, "tri_attn_block")
    B, N = int(z4.shape[0]), int(z4.shape[1])
    m, mdt, mframe = _pair_mask(mask, z4, ending)
    wqkvg, wb, wo = _wpack(W, z.dtype, z.device)
    dt = L.DT_BF16 if z.dtype == torch.bfloat16 else L.DT_F32
    need = L.lib().fpf_triattn_block_workspace_bytes(B, N, 0, W.C, W.H, W.D, dt)
    wkey = str(z.device)
    ws = W._ws.get(wkey)
    if ws is None or ws.numel() < need:
        ws = W._ws[wkey] = torch.empty(need, dtype=torch.uint8, device=z.device)
    out = z4 if residual else torch.empty_like(z4)
    a = L.TriattnBlockArgs(abi_version=L.ABI_VERSION, dtype=dt, B=B, N=N, C=W.C, H=W.H, D=W.D, z=L.ptr(z4), mask=L.ptr(m), mask_dtype=mdt,
                           ln_w=L.ptr(W.ln_w), ln_b=L.ptr(W.ln_b), eps=W.eps, w_qkvg=L.ptr(wqkvg), w_b=L.ptr(wb), w_o=L.ptr(wo),
                           ending=1 if ending else 0, residual=1 if residual else 0, out=L.ptr(out), scale=float(scale or 0.0),
                           workspace=L.ptr(ws), workspace_bytes=ws.numel(), mask_frame=mframe)
    try:
        L.call("fpf_triattn_block_fwd", a, L.stream_ptr(z.device))
    except L.LibError as e:
        raise Unsupported("lib:" + e.kind, e.msg) from None
    if residual:
        return z
    return out if z.dim() == 4 else out[0]


def tri_attn_block_chunked(z, W, mask=None, *, ending=False, residual=False, chunk=256, scale=None, word="big", **_unused):
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
    wqkvg, wb, wo = _wpack(W, z.dtype, z.device)
    rows = min(chunk, N)
    lib = L.lib()
    need = lib.fpf_triattn_block_workspace_bytes(B, N, rows, W.C, W.H, W.D, L.DT_BF16)
    key = (str(z.device), "chunked")
    ws = W._ws.get(key)
    if ws is None or ws.numel() < need:
        ws = W._ws[key] = torch.empty(need, dtype=torch.uint8, device=z.device)
    bkey = (str(z.device), "bias")
    bias = W._ws.get(bkey)
    if bias is None or bias.numel() < B * W.H * N * N:
        bias = W._ws[bkey] = torch.empty(B * W.H * N * N, dtype=torch.float32, device=z.device)
    stream = L.stream_ptr(z.device)
    ab = L.TriattnBiasArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, B=B, N=N, C=W.C, H=W.H, D=W.D, z=L.ptr(z4), ln_w=L.ptr(W.ln_w),
                           ln_b=L.ptr(W.ln_b), eps=W.eps, w_qkvg=L.ptr(wqkvg), w_b=L.ptr(wb), ending=1 if ending else 0, bias=L.ptr(bias))
    try:
        L.call("fpf_triattn_bias_fwd", ab, stream)
    except L.LibError as e:
        raise Unsupported("lib:" + e.kind, e.msg) from None
    out = z4 if residual else torch.empty_like(z4)
    for r0 in range(0, N, rows):
        a = L.TriattnBlockArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, B=B, N=N, C=W.C, H=W.H, D=W.D, z=L.ptr(z4), mask=L.ptr(m),
                               mask_dtype=mdt, ln_w=L.ptr(W.ln_w), ln_b=L.ptr(W.ln_b), eps=W.eps, w_qkvg=L.ptr(wqkvg), w_b=L.ptr(wb),
                               w_o=L.ptr(wo), ending=1 if ending else 0, residual=1 if residual else 0, out=L.ptr(out),
                               scale=float(scale or 0.0), workspace=L.ptr(ws), workspace_bytes=ws.numel(), row0=r0, rows=min(rows, N - r0),
                               bias_in=L.ptr(bias), mask_frame=mframe)
        try:
            L.call("fpf_triattn_block_fwd", a, stream)
        except L.LibError as e:
            raise Unsupported("lib:" + e.kind, e.msg) from None
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
    C, NH = int(w_out.shape[0]), int(w_out.shape[1])
    if w_ab is not None:
        if tuple(w_ab.shape) != (2 * NH, C):
            raise Unsupported("w_ab-shape", str(tuple(w_ab.shape)))
        blocks = {nm: w_ab[i * NH:(i + 1) * NH] for i, nm in enumerate(ab_split)}
        w_a, w_b = blocks["a"], blocks["b"]
    for nm, t in (("w_a", w_a), ("w_b", w_b)):
        if t is None or tuple(t.shape) != (NH, C):
            raise Unsupported(nm + "-shape", str(None if t is None else tuple(t.shape)))
    return TransitionWeights(_TR.pack(w_o=w_out, w_a=w_a, w_b=w_b, ln_w=ln_w, ln_b=ln_b, eps=eps, device=device))


def transition(x, T, *, residual=False, out=None, mask=None, word="fast", **_unused):
    """y = W_out(silu(W_a n) * W_b n), n = LN(x) in-kernel; x + y when residual; ``out`` may be x (in place)."""
    try:
        y, _sel = _TR.transition(x, T.W, word=word, residual=residual, mask=mask, out=out)
    except F.Refusal as e:
        raise Unsupported(e.kind, e.detail) from None
    return y

"""Transition face: y = W_o(silu(W_a n) * (W_b n)), n = LayerNorm(x), optional row mask and residual folded in the kernel,
served by libfpf_hip's ``fpf_transition_fwd`` (one launch; the hidden never reaches HBM).

Mirrors common/opt_core/opt_core/kernels/transition/__init__.py: ``pack(*, w_o, w_a=None, w_b=None, w_ab=None, ln_w=None,
ln_b=None, eps=1e-5, device=None) -> Weights`` (:1011), ``Weights`` (:928; operand packs built once per weight set and dtype)
``select(word, *, c, hidden, n_tokens=None, dtype="bf16", ...)`` (:509) and ``transition(x, W, *, word, residual=False, x_ln=None,
mask=None, binary_mask=None, out=None, n_tokens=None, family="pair", ...) -> (y, Selection)`` (:1074).  ``out`` may be ``x`` itself
(in place).  ``x_ln`` (the caller's own LayerNorm output of x, the exact-candidate construction) is projected in place of the
in-kernel LayerNorm on the bf16 row; the fp32 row refuses it by name.
"""
import torch

from .. import _face as F
from .. import _lib as L
from .. import cells as CELLS

Refusal, Selection = F.Refusal, F.Selection


class Weights(object):
    """Canonical transition weights: w_a / w_b [hidden, c], w_o [c, hidden], LayerNorm ln_w / ln_b [c] (None = no affine),
    eps.  Device operand packs (bf16 or fp32 contiguous copies) are built on first use per (device, dtype) and kept."""

    def __init__(self, w_a, w_b, w_o, ln_w, ln_b, eps, device):
        self.c, self.hidden = int(w_o.shape[0]), int(w_o.shape[1])
        if tuple(w_a.shape) != (self.hidden, self.c) or tuple(w_b.shape) != (self.hidden, self.c):
            raise Refusal("weights:shapes:%s:%s:%s" % (tuple(w_a.shape), tuple(w_b.shape), tuple(w_o.shape)), None, F.ROW_STOCK)
        dev = device if device is not None else w_o.device
        self.w_a, self.w_b, self.w_o = (t.detach().to(dev) for t in (w_a, w_b, w_o))
        self.ln_w = None if ln_w is None else ln_w.detach().to(dev).float().contiguous()
        self.ln_b = None if ln_b is None else ln_b.detach().to(dev).float().contiguous()
        self.eps = float(eps)
        self.device = dev
        self._packs = {}

    def pack_for(self, dtype, device):
        key = (str(device), dtype)
        p = self._packs.get(key)
        if p is None:
            with torch.no_grad():
                p = tuple(t.to(device=device, dtype=dtype).contiguous() for t in (self.w_a, self.w_b, self.w_o))
                p = p + (None if self.ln_w is None else self.ln_w.to(device),
                         None if self.ln_b is None else self.ln_b.to(device))
            self._packs[key] = p
        return p


def pack(*, w_o, w_a=None, w_b=None, w_ab=None, ln_w=None, ln_b=None, eps=1e-5, device=None):
    """w_ab [2*hidden, c] = rows a (silu branch) then b -- the Boltz fc1|fc2 concatenation."""
    if w_ab is not None:
        h = int(w_ab.shape[0]) // 2
        w_a, w_b = w_ab[:h], w_ab[h:]
    if w_a is None or w_b is None:
        raise Refusal("weights:missing_w_a_w_b", None, F.ROW_STOCK)
    return Weights(w_a, w_b, w_o, ln_w, ln_b, eps, device)


def _arch_of(cc, device):
    if cc is not None:
        return F.arch_word(cc)
    if device is not None:
        return F.arch_word(torch.device(device))
    return F.arch_word(torch.device("cuda")) if torch.cuda.is_available() else "cpu"


def select(word, *, c, hidden, n_tokens=None, dtype="bf16", direction="fwd", timing="eager", family="pair", residual=False, mask=False,
           cc=None, device=None, stack=None, capture=False, rows_count=None, ln_given=False, form="swiglu"):
    """Pure: the row serving a transition of this class, or Refusal by name (common/opt_core/opt_core/kernels/transition/__init__.py:509).
    ``cc`` / ``device`` name the card (the current device when both are None); ``n_tokens`` (the pair tensor's N) names the
    measured cell.  ``ln_given`` (the caller's own LayerNorm output, the exact-candidate construction) is served by the bf16 row
    and refused by name on the fp32 row; any ``form`` other than swiglu is refused by name; ``timing`` / ``capture`` / ``stack`` / ``rows_count`` / ``residual`` / ``mask`` do not change the
    answer (the kernel folds the residual and the row mask and is capture-safe)."""
    w = F.word_base(word)
    if str(direction) not in ("fwd", "forward"):
        raise Refusal("no_backward", w, F.ROW_STOCK, "forward only")
    if form != "swiglu":
        raise Refusal("form:%s" % form, w, F.ROW_STOCK, "the kernel computes the SwiGLU transition")
    dw = F.dtype_of(dtype)
    c, hidden = int(c), int(hidden)
    cell = "%s|%s|%s_c%d_n%d|eager|fwd" % (CELLS.CC, dw, family, c, hidden // max(c, 1))
    if n_tokens is not None and hidden % c == 0 and family == "pair":
        cell = CELLS.transition_key(dw, c, hidden // c, n_tokens)
    sel = F.resolve(w, dw, _arch_of(cc, device), "transition", cell=cell)
    if sel.row == F.ROW_FAST and (c != 128 or hidden % 32):
        raise Refusal("shape:c%dh%d" % (c, hidden), sel.row, F.ROW_F32, "the bf16 kernel serves c = 128, hidden % 32 == 0")
    if sel.row == F.ROW_F32 and c > 384:
        raise Refusal("shape:c%d" % c, sel.row, F.ROW_STOCK, "the fp32 kernel serves c <= 384")
    if ln_given and sel.row != F.ROW_FAST:
        raise Refusal("ln_given", sel.row, F.ROW_STOCK, "the fp32 row normalises in-kernel; the caller's x_ln is taken by the bf16 row")
    return sel


def transition(x, W, *, word, residual=False, x_ln=None, mask=None, binary_mask=None, out=None, n_tokens=None, family="pair", timing="eager",
               capture=False, stack=None, form="swiglu", cc=None, selection=None, pair_bias=None):
    """y = W_o(silu(W_a n) * (W_b n)), n = LayerNorm(x) in-kernel -> (y, Selection); x + y when ``residual``; ``mask`` one value
    per row of x (any values: the update is multiplied by it before the residual add, so ``binary_mask`` changes nothing);
    ``out`` may be x (in place).  The hidden is fp32 and rounded to bf16 once (silu(a) * b) before the output projection.

    ``pair_bias`` (bf16 pair tensor x [B, N, N, 128] or [N, N, 128]): a dict ``w_z`` [H, 128] (H <= 32), ``out`` [B, H, N, N] fp32 |
    bf16 (unit key stride, one row pitch), optional ``ln_w`` / ``ln_b`` [128] and ``eps`` -- the single track's pair bias
    LN(row) . w_z[h] of the rows this call writes, computed in the same kernel (boltz2/opt/forward/pairfuse/bz_pairfuse.py:18-20
    runs it as its own pass over the resident z; the values equal ``attn.apb_core.pair_bias_producer`` on the written z)."""
    c = int(x.shape[-1])
    if c != W.c:
        raise Refusal("c:%d!=%d" % (c, W.c), word, F.ROW_STOCK)
    if n_tokens is None and x.dim() >= 3:
        n_tokens = int(x.shape[-2])
    sel = selection or select(word, c=W.c, hidden=W.hidden, n_tokens=n_tokens, dtype=x.dtype, family=family, residual=residual,
                              mask=mask is not None, cc=cc if cc is not None else x, stack=stack, capture=capture, ln_given=x_ln is not None,
                              form=form, timing=timing)
    rows = x.numel() // c
    if not x.is_contiguous():
        raise Refusal("stride", sel.row, F.ROW_STOCK, "x must be contiguous")
    F.check_device("transition", sel.row, x.device, out=out)
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise Refusal("out", sel.row, F.ROW_STOCK, "out must be contiguous, x's shape and dtype")
    m = None
    if mask is not None:
        m = mask.reshape(-1)
        if m.numel() != rows:
            raise Refusal("mask_rows", sel.row, F.ROW_STOCK, "one mask value per row")
        m = m.to(device=x.device, dtype=torch.float32).contiguous()
    if x_ln is not None and (x_ln.shape != x.shape or x_ln.dtype != torch.bfloat16 or not x_ln.is_contiguous() or x_ln.device != x.device):
        raise Refusal("x_ln", sel.row, F.ROW_STOCK, "x_ln must be a contiguous bf16 tensor of x's shape on x's device")
    wa, wb, wo, lw, lb = W.pack_for(x.dtype, x.device)
    a = L.TransitionArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16 if x.dtype == torch.bfloat16 else L.DT_F32, c=c, hidden=W.hidden,
                         rows=rows, x=L.ptr(x), out=L.ptr(out), ln_w=L.ptr(lw), ln_b=L.ptr(lb), eps=W.eps, w_a=L.ptr(wa), w_b=L.ptr(wb),
                         w_o=L.ptr(wo), row_mask=L.ptr(m), residual=1 if residual else 0, x_ln=L.ptr(x_ln))
    keep = _pair_bias_args(a, x, pair_bias, sel) if pair_bias is not None else None
    L.call("fpf_transition_fwd", a, L.stream_ptr(x.device))
    del keep
    return out, sel


def _pair_bias_args(a, x, pb, sel):
    """Fills the pair-bias fields of ``a`` from the ``pair_bias`` dict; returns the device tensors the call reads (kept alive by
    the caller until the launch)."""
    if x.dtype != torch.bfloat16 or sel.row != F.ROW_FAST:
        raise Refusal("pair_bias:precision", sel.row, F.ROW_STOCK, "the pair bias is projected by the bf16 transition")
    x4 = x if x.dim() == 4 else x.unsqueeze(0)
    if x4.dim() != 4 or int(x4.shape[1]) != int(x4.shape[2]) or int(x4.shape[3]) != 128:
        raise Refusal("pair_bias:not_pair", sel.row, F.ROW_STOCK, "x must be a pair tensor [B, N, N, 128] (got %s)" % (tuple(x.shape),))
    B, N = int(x4.shape[0]), int(x4.shape[1])
    w_z, bias = pb.get("w_z"), pb.get("out")
    if w_z is None or bias is None:
        raise Refusal("pair_bias:args", sel.row, F.ROW_STOCK, "pair_bias needs w_z and out")
    H = int(w_z.shape[0])
    if w_z.dim() != 2 or int(w_z.shape[1]) != 128 or not 1 <= H <= 32:
        raise Refusal("pair_bias:w_z", sel.row, F.ROW_STOCK, "w_z [H <= 32, 128] (got %s)" % (tuple(w_z.shape),))
    if (tuple(bias.shape) != (B, H, N, N) or bias.dtype not in (torch.float32, torch.bfloat16) or bias.device != x.device
            or bias.stride(3) != 1 or bias.stride(1) != N * bias.stride(2) or bias.stride(0) != H * bias.stride(1)):
        raise Refusal("pair_bias:out", sel.row, F.ROW_STOCK, "out must be an fp32 | bf16 [B, H, N, N] on x's device with rows of one pitch")
    wz = w_z.to(device=x.device, dtype=torch.bfloat16).contiguous()
    lw = None if pb.get("ln_w") is None else pb["ln_w"].to(device=x.device, dtype=torch.float32).contiguous()
    lb = None if pb.get("ln_b") is None else pb["ln_b"].to(device=x.device, dtype=torch.float32).contiguous()
    a.w_z, a.z_ln_w, a.z_ln_b, a.z_eps, a.z_heads = L.ptr(wz), L.ptr(lw), L.ptr(lb), float(pb.get("eps", 1e-5)), H
    a.pair_n, a.z_bias, a.z_bias_ld = N, L.ptr(bias), int(bias.stride(2))
    a.z_bias_dtype = L.DT_F32 if bias.dtype == torch.float32 else L.DT_BF16
    return wz, lw, lb


def pair_transition_chunked(x, W, *, chunk, row_dim=-3, word="big", residual=False, mask=None, out=None, fp32="passthrough", selection=None):
    """Row-chunked pair transition (common/opt_core/opt_core/mem/chunk.py:370 ``pair_transition_chunked``): ``transition`` on
    blocks of ``chunk`` rows of ``x [..., I, J, C]`` (``row_dim`` = the I axis, the only one served), one ``fpf_transition_fwd``
    launch per block and leading index -> (y, Selection).  The statement is per position, so the result equals the unchunked
    transition's bitwise; the kernel keeps the 4c hidden on chip, so a block bounds nothing but the launch extent (the
    reference's blocks bound its [.., I, J, 4C] intermediates).  ``residual`` / ``out`` (x itself for in place) / ``mask`` (one
    value per position, [..., I, J]) as in ``transition``.  An fp32 x runs unchunked for ``fp32`` = ``"passthrough"`` (the
    reference's guard) or ``"band"`` (the unchunked result meets it) and is refused for ``"refuse"``."""
    if str(fp32) not in ("passthrough", "band", "refuse"):
        raise ValueError("fp32 must be passthrough | band | refuse (got %r)" % (fp32,))
    chunk = int(chunk)
    if chunk <= 0:
        raise ValueError("chunk must be positive (got %d)" % chunk)
    if x.dim() < 3:
        raise Refusal("not_pair_shaped", F.word_base(word), F.ROW_STOCK, "x has rank %d, expected [..., I, J, C]" % x.dim())
    if int(row_dim) not in (-3, x.dim() - 3):
        raise Refusal("row_dim:%s" % row_dim, F.word_base(word), F.ROW_STOCK, "the row blocks run along the I axis (row_dim -3)")
    sel = selection or select(word, c=int(x.shape[-1]), hidden=W.hidden, n_tokens=int(x.shape[-2]), dtype=x.dtype, cc=x, residual=residual,
                              mask=mask is not None)
    if sel.row != F.ROW_FAST:
        if str(fp32) == "refuse":
            raise Refusal("fp32_site", sel.row, F.ROW_STOCK, "an fp32 transition is not chunked (fp32='refuse')")
        return transition(x, W, word=word, residual=residual, mask=mask, out=out, selection=sel)
    if not x.is_contiguous():
        raise Refusal("stride", sel.row, F.ROW_STOCK, "x must be contiguous")
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise Refusal("out", sel.row, F.ROW_STOCK, "out must be contiguous, x's shape and dtype")
    I, J, C = (int(s) for s in x.shape[-3:])
    x3, o3 = x.view(-1, I, J, C), out.view(-1, I, J, C)
    m3 = None
    if mask is not None:
        if mask.numel() != x.numel() // C:
            raise Refusal("mask_rows", sel.row, F.ROW_STOCK, "one mask value per position")
        m3 = mask.reshape(-1, I, J)
    for l in range(x3.shape[0]):
        for i0 in range(0, I, chunk):
            i1 = min(i0 + chunk, I)
            transition(x3[l, i0:i1], W, word=word, residual=residual, mask=None if m3 is None else m3[l, i0:i1], out=o3[l, i0:i1],
                       selection=sel)
    return out, sel

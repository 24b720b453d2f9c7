"""LayerNorm face: F.layer_norm semantics over the last dimension, served by libfpf_hip's ``fpf_layernorm_fwd``.

Mirrors common/opt_core/opt_core/kernels/ln/__init__.py:836 (``layer_norm(x, normalized_shape, weight, bias, eps, *, word, ...)
-> (y, Selection)``) and :408 (``select(cc, dtype, cell, n_tokens, *, word, ...)``); forms: fp32 (fp32 in / out), bf16 (bf16 in / out), bf16w (bf16 in, fp32 out: ``out_dtype=torch.float32``),
bf16o (bf16 in, fp32 gamma / beta, bf16 out).  gamma / beta are read as fp32 whatever their dtype (cast once per call here when
they are not fp32 already).
"""
import torch

from .. import _face as F
from .. import _lib as L

Refusal, Selection = F.Refusal, F.Selection


def select(cc, dtype, cell, n_tokens, *, word, widen=False, out=None, timing="eager", pass_="fwd", prefer=None, stack=None, capture=False,
           C=None, has_nvrtc=None, rows=None, has_triton=None, has_esm=None, aligned=True, config=None, affine=True):
    """Pure: the row that serves a LayerNorm call of this dtype on this card, or Refusal by name (ln/__init__.py:408).  ``C``
    (the normalised width) bounds the row; ``widen`` (bf16 x with fp32 parameters) and ``out`` ('bf16': the bf16o form) are
    forms of the same row; ``pass_`` other than fwd is refused.  ``cell`` names the measured cell; ``timing`` / ``capture`` /
    ``stack`` / ``rows`` / ``aligned`` / ``affine`` / the library-presence flags do not change the answer."""
    w = F.word_base(word)
    if pass_ != "fwd":
        raise Refusal("no_backward", w, F.ROW_STOCK, "forward only")
    sel = F.resolve(w, F.dtype_of(dtype), F.arch_word(cc), "ln", cell="ln:c%s" % C)
    F.narrow(sel, w, prefer)
    F.no_config(config, sel.row)
    if C is not None and (int(C) > 1024 or int(C) % 8):
        raise Refusal("cols:%d" % int(C), sel.row, F.ROW_STOCK, "cols must be a multiple of 8 and <= 1024")
    return sel


def _f32(t, C, dev):
    if t is None:
        return None
    t = t.detach()
    if t.dtype != torch.float32 or t.device != dev or not t.is_contiguous():
        t = t.to(device=dev, dtype=torch.float32).contiguous()
    if t.numel() != C:
        raise Refusal("param_shape", None, F.ROW_STOCK, str(tuple(t.shape)))
    return t


def layer_norm(x, normalized_shape, weight=None, bias=None, eps=1e-5, *, word=None, selection=None, n_tokens=None, cell=None, prefer=None,
               capture=False, out_dtype=None, cache=None, out=None):
    """F.layer_norm semantics over the last dimension -> (y, Selection).  ``word`` or ``selection`` is required."""
    C = int(normalized_shape[-1]) if isinstance(normalized_shape, (tuple, list)) else int(normalized_shape)
    if x.shape[-1] != C:
        raise Refusal("normalized_shape", None, F.ROW_STOCK, "%s vs %s" % (tuple(x.shape), C))
    rows_ = x.numel() // C if C else 0
    sel = selection or select(x, x.dtype, cell, n_tokens if n_tokens is not None else int(round(rows_ ** 0.5)), word=word, prefer=prefer,
                              capture=capture, C=C, rows=rows_, widen=x.dtype == torch.bfloat16 and weight is not None and weight.dtype == torch.float32,
                              out="bf16" if out_dtype == torch.bfloat16 else None)
    F.check_device("ln", sel.row, x.device, out=out)
    odt = out_dtype or x.dtype
    if odt not in (torch.bfloat16, torch.float32):
        raise Refusal("out_dtype:%s" % odt, sel.row)
    rows = x.numel() // C if C else 0
    x2 = x.reshape(rows, C)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    y = out if out is not None else torch.empty(x.shape, dtype=odt, device=x.device)
    if y.dtype != odt or y.shape != x.shape or not y.is_contiguous():
        raise Refusal("out", sel.row, F.ROW_STOCK, "out must be a contiguous %s tensor of x's shape" % odt)
    w_, b_ = _f32(weight, C, x.device), _f32(bias, C, x.device)
    a = L.LnArgs(abi_version=L.ABI_VERSION, dtype_in=L.DT_BF16 if x.dtype == torch.bfloat16 else L.DT_F32,
                 dtype_out=L.DT_BF16 if odt == torch.bfloat16 else L.DT_F32, cols=C, rows=rows, x=L.ptr(x2), x_row_stride=x2.stride(0),
                 y=L.ptr(y), y_row_stride=C, gamma=L.ptr(w_), beta=L.ptr(b_), eps=float(eps))
    L.call("fpf_layernorm_fwd", a, L.stream_ptr(x.device))
    return y, sel

"""Triangle-attention face (the op), served by libfpf_hip's ``fpf_triattn_fwd``.

Mirrors common/opt_core/opt_core/kernels/triattn/__init__.py: the op (:3-8)

    out[b,n,h,i,:] = softmax_j( scale*q[b,n,h,i,:].k[b,n,h,j,:] + bias[b,0,h,i,j]  (-inf where mask[b,n,0,0,j] is False) ) @ v[b,n,h,j,:]
    q/k/v [B,N,H,S,D], bias [B,1,H,S,S] (fp32 or bf16, shared over the N rows), mask [B,N,1,1,S] (bool / any dtype, nonzero = attend),
    out [B,N,H,S,D] in q.dtype; a fully-masked row yields the uniform average of v,

``Refusal`` (:129), ``Selection``, ``select(cc, dtype, head_dim, heads, n_tokens, direction="fwd", *, word)`` (:454) and
``triangle_attention(q, k, v, bias, mask=None, scale=None, *, word, ...)`` (:1094).  Strided views are served as they are
(stride(-1) == 1): the ending node's transposed q/k/v views need no copy.
"""
import math

import torch

from .. import _face as F
from .. import _lib as L
from .. import cells as CELLS

Refusal, Selection = F.Refusal, F.Selection


def select(arch, dtype, head_dim, heads, n_tokens, direction="fwd", *, word):
    """Pure: the row serving a triangle-attention call of this class on this device word, or Refusal by name."""
    if direction not in ("fwd", "forward", "inference", "start", "starting", "end", "ending"):
        raise Refusal("direction:%s" % direction, word, F.ROW_STOCK, "forward only")
    sel = F.resolve(word, F.dtype_word(dtype), arch, "triattn", cell=CELLS.triattn_key(F.dtype_word(dtype), head_dim, heads, n_tokens))
    if sel.row == F.ROW_FAST and head_dim != 32:
        raise Refusal("no_row:head_dim%d" % head_dim, sel.row, F.ROW_F32, "the bf16 core serves head_dim 32")
    if sel.row == F.ROW_F32 and head_dim not in (16, 32, 64):
        raise Refusal("no_row:head_dim%d" % head_dim, sel.row, F.ROW_STOCK, "the fp32 core serves head_dim 16 | 32 | 64")
    return sel


def _strides(t, n):
    s = list(t.stride())
    if len(s) != n:
        raise Refusal("rank", None, F.ROW_STOCK, str(tuple(t.shape)))
    return s


def triangle_attention(q, k, v, bias, mask=None, scale=None, *, word, selection=None, out=None, **_unused):
    """Serve the op; returns the output tensor.  Refusal by name before any launch."""
    if q.dim() != 5 or k.shape != q.shape or v.shape != q.shape:
        raise Refusal("shape", word, F.ROW_STOCK, "q/k/v must be [B,N,H,S,D] of one shape")
    B, N, H, S, D = q.shape
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise Refusal("dtype_mix", word, F.ROW_STOCK)
    sel = selection or select(F.device_word(q), q.dtype, D, H, S, word=word)
    # v stored transposed ([B,N,H,D,S] storage viewed as [B,N,H,S,D], as the block prologue returns it) is served as it is by
    # the bf16 core (v_layout 1); every other operand needs a contiguous head_dim
    v_t = v.stride(-1) != 1 and v.stride(-2) == 1 and D > 1
    if q.stride(-1) != 1 or k.stride(-1) != 1 or (v.stride(-1) != 1 and not v_t):
        raise Refusal("stride", sel.row, F.ROW_STOCK, "head_dim must be contiguous")
    if v_t and sel.row != F.ROW_FAST:
        raise Refusal("stride:v_transposed", sel.row, F.ROW_FAST, "the fp32 core takes v with a contiguous head_dim")
    if bias.dim() != 5 or tuple(bias.shape) != (B, 1, H, S, S) or bias.stride(-1) != 1:
        raise Refusal("bias_shape", sel.row, F.ROW_STOCK, str(tuple(bias.shape)))
    if bias.dtype not in (torch.float32, torch.bfloat16):
        raise Refusal("bias_dtype:%s" % bias.dtype, sel.row, F.ROW_STOCK)
    m = None
    mdt = L.DT_U8
    if mask is not None:
        m = mask.reshape(B, N, S) if mask.numel() == B * N * S else None
        if m is None:
            raise Refusal("mask_shape", sel.row, F.ROW_STOCK, str(tuple(mask.shape)))
        if m.dtype == torch.bool:
            m = m.view(torch.uint8)
        elif m.dtype != torch.float32:
            m = (m != 0).view(torch.uint8)
        else:
            mdt = L.DT_F32
    if out is None:
        out = torch.empty((B, N, H, S, D), dtype=q.dtype, device=q.device)
    sc = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    a = L.TriattnArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16 if q.dtype == torch.bfloat16 else L.DT_F32, B=B, N=N, H=H, S=S, D=D,
                      q=L.ptr(q), k=L.ptr(k), v=L.ptr(v), bias=L.ptr(bias), bias_dtype=L.DT_F32 if bias.dtype == torch.float32 else L.DT_BF16,
                      mask=L.ptr(m), mask_dtype=mdt, out=L.ptr(out), scale=sc)
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("out_stride", out)):
        getattr(a, name)[:] = _strides(t, 5)
    if v_t:
        vs = _strides(v, 5)
        a.v_layout = 1
        a.v_stride[:] = [vs[0], vs[1], vs[2], vs[4], vs[3]]
    bs = _strides(bias, 5)
    a.bias_stride[:] = [bs[0], bs[2], bs[3], bs[4]]
    if m is not None:
        a.mask_stride[:] = _strides(m, 3)
    L.call("fpf_triattn_fwd", a, L.stream_ptr(q.device))
    return out

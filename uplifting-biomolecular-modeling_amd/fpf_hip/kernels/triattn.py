"""Triangle-attention face (the op), served by libfpf_hip's ``fpf_triattn_fwd``.

Mirrors common/opt_core/opt_core/kernels/triattn/__init__.py: the op (:3-8)

    out[b,n,h,i,:] = softmax_j( scale*q[b,n,h,i,:].k[b,n,h,j,:] + bias[b,0,h,i,j]  (-inf where mask[b,n,0,0,j] is False) ) @ v[b,n,h,j,:]
    q/k/v [B,N,H,S,D], bias [B,1,H,S,S] (fp32 or bf16, shared over the N rows), mask [B,N,1,1,S] (bool / any dtype, nonzero = attend),
    out [B,N,H,S,D] in q.dtype; a fully-masked row yields the uniform average of v,

``Refusal`` (:129), ``Selection``, ``select(cc, dtype, head_dim, heads, n_tokens, direction="fwd", *, word, prefer=None, stack=None,
config=None, ...)`` (:454), ``admits(row, cc, dtype, head_dim, heads, n_tokens, direction="fwd", *, stack=None, position_stride=None)``
(:305) and ``triangle_attention(q, k, v, bias, mask=None, scale=None, *, word, prefer=None, stock=None, config=None, selection=None,
form=None)`` (:1094).  ``cc`` is a capability ((9, 5) / "9.5" for an MI355X under ROCm torch), an arch name ("gfx950") or a device.
Strided views are served as they are (stride(-1) == 1): the ending node's transposed q/k/v views need no copy.
"""
import math

import torch

from .. import _face as F
from .. import _lib as L
from .. import cells as CELLS

Refusal, Selection = F.Refusal, F.Selection
ROW_NAMES = (F.ROW_FAST, F.ROW_F32)
_DIRECTIONS = ("fwd", "forward", "inference", "start", "starting", "end", "ending")


def admits(row, cc, dtype, head_dim, heads, n_tokens, direction="fwd", *, stack=None, position_stride=None):
    """(True, "ok") when ``row``'s static envelope admits the call, else (False, <refusal word>) -- pure, no launch."""
    if row not in ROW_NAMES:
        return False, "unknown_row:%s" % row
    if F.arch_word(cc) != F.ARCH:
        return False, "arch:%s" % F.arch_word(cc)
    if str(direction) not in _DIRECTIONS:
        return False, "direction:%s" % direction
    dw = F.dtype_of(dtype)
    if row == F.ROW_FAST and (dw != "bf16" or int(head_dim) != 32):
        return False, "dtype:%s" % dw if dw != "bf16" else "no_row:head_dim%d" % int(head_dim)
    if row == F.ROW_F32 and (dw != "fp32" or int(head_dim) not in (16, 32, 64)):
        return False, "dtype:%s" % dw if dw != "fp32" else "no_row:head_dim%d" % int(head_dim)
    return True, "ok"


def select(cc, dtype, head_dim, heads, n_tokens, direction="fwd", *, word, prefer=None, stack=None, config=None, position_stride=None,
           form=None, exact_stack=None, lib=None):
    """Pure: the row serving a triangle-attention call of this class on this device, or Refusal by name.  ``prefer`` narrows a
    tier word's candidates; ``config`` (a launch setting) is refused by name; ``stack`` / ``form`` / ``exact_stack`` / ``lib`` /
    ``position_stride`` do not change the answer (the kernels take 64-bit offsets and any strided q / k / v view)."""
    w = F.word_base(word)
    if str(direction) not in _DIRECTIONS:
        raise Refusal("direction:%s" % direction, w, F.ROW_STOCK, "forward only")
    dw = F.dtype_of(dtype)
    sel = F.resolve(w, dw, F.arch_word(cc), "triattn", cell=CELLS.triattn_key(dw, head_dim, heads, n_tokens))
    F.narrow(sel, w, prefer)
    F.no_config(config, sel.row)
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


def triangle_attention(q, k, v, bias, mask=None, scale=None, *, word, prefer=None, stock=None, config=None, selection=None, form=None,
                       out=None):
    """Serve the op; returns the output tensor.  Refusal by name before any launch.  ``stock`` (the kit's own stock callable) is
    never called here: this face serves only its own rows, and the stock row is the caller's call.  ``out`` (an extension of this
    package): a caller-given [B, N, H, S, D] output."""
    if q.dim() != 5 or k.shape != q.shape or v.shape != q.shape:
        raise Refusal("shape", word, F.ROW_STOCK, "q/k/v must be [B,N,H,S,D] of one shape")
    B, N, H, S, D = q.shape
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise Refusal("dtype_mix", word, F.ROW_STOCK)
    sel = selection or select(q, q.dtype, D, H, S, word=word, prefer=prefer, config=config, form=form)
    F.check_device("triattn", sel.row, q.device, k=k, v=v, bias=bias, out=out)
    if mask is not None and mask.device != q.device:
        mask = mask.to(q.device)
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
    elif tuple(out.shape) != (B, N, H, S, D) or out.dtype != q.dtype or out.stride(-1) != 1:
        raise Refusal("out", sel.row, F.ROW_STOCK, "out must be [B,N,H,S,D] in q's dtype with a contiguous head_dim")
    sc = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    dt = L.DT_BF16 if q.dtype == torch.bfloat16 else L.DT_F32
    # bf16 at head_dim 32: a workspace of the staging size routes the call onto the block-layout core (V^T, bias and mask
    # restaged into its layout, q and k read in place; the library keeps the op core when the strides do not allow it)
    stage = L.lib().fpf_triattn_stage_bytes(B, N, H, S, D, dt)
    ws = F.scratch(q.device, stage, kind="op") if stage else None
    a = L.TriattnArgs(abi_version=L.ABI_VERSION, dtype=dt, B=B, N=N, H=H, S=S, D=D,
                      q=L.ptr(q), k=L.ptr(k), v=L.ptr(v), bias=L.ptr(bias), bias_dtype=L.DT_F32 if bias.dtype == torch.float32 else L.DT_BF16,
                      mask=L.ptr(m), mask_dtype=mdt, out=L.ptr(out), scale=sc, workspace=L.ptr(ws), workspace_bytes=0 if ws is None else ws.numel())
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

"""Attention with a pair bias over libfpf_hip (``fpf_apb_fwd``; the producer ``fpf_apb_bias_fwd``): the Pairformer single track's
AttentionPairBias and the token attention of a sample batch sharing one bias.

Mirrors common/opt_core/opt_core/attn/apb_core.py: ``Unsupported(event, detail)`` (:45), ``census()`` (:63) and

    out = pair_bias_attention(q, k, v, pair_bias, key_mask=None, *, gate=None, num_samples=None, num_heads=None, layout="rows",
                              out=None, scale=None, inf=1e9)                                                              (:89)

    out[s, i, h*D:(h+1)*D] = sigmoid(gate[s, i, hD..]) * softmax_j( scale q.k + pair_bias[s|0, h, i, j] - inf (key_mask[s|0, j] == 0) ) @ v

Layouts as in the reference (:13-18): "rows" = q, k, v, gate 2-D [S*N, H*D] row blocks with unit column stride (typically the
column slices of one fused projection output), "shnd" = q, k, v [S, H, N, D] with innermost stride 1, gate [S, N, H*D] or
[S, N, H, D].  Both are served IN PLACE through strides.  pair_bias [H, N, NK] or [SB, H, N, NK] (SB in {1, S}, leading singleton
dims allowed), fp32 or bf16, unit key stride; key_mask [NK], [1, NK] or [S, NK], any dtype, nonzero = attend.  A masked key adds
-inf (a sample whose keys are all masked gives the uniform mean of v over all keys, never NaN), so ``inf`` must be finite and is
otherwise not used.  Refusals raise ``Unsupported`` by name BEFORE any launch.  fp32 arithmetic throughout (the stock single
track runs with autocast off), for fp32 or bf16 storage.

Also here: ``pair_bias_producer`` (the kernels/apb "producer" boundary: bias = Linear_{c_z -> H}(LayerNorm(z)) head-major, in one
pass over bf16 z) and ``attention_pair_bias_module`` (the whole AttentionPairBias module, attentionv2.py:62-111: the q|k|v|g and
output projections are plain GEMMs through torch, the core and the producer are the HIP kernels).
"""
import math
import threading

import torch

from .. import _lib as L

LAYOUTS = ("rows", "shnd")
HEAD_DIMS = (16, 24, 32, 48, 64)
CENSUS = {"served": 0, "refused": {}, "by_shape": {}}
_LOCK = threading.Lock()


class Unsupported(Exception):
    """An input outside the served domain, refused by name before any work (``.event``, ``.detail``)."""

    def __init__(self, event, detail=""):
        Exception.__init__(self, "%s: %s" % (event, detail) if detail else event)
        self.event, self.detail = event, detail


def _book(event, key=None):
    with _LOCK:
        if event is None:
            CENSUS["served"] += 1
            if key is not None and (key in CENSUS["by_shape"] or len(CENSUS["by_shape"]) < 32):
                CENSUS["by_shape"][key] = CENSUS["by_shape"].get(key, 0) + 1
        else:
            CENSUS["refused"][event] = CENSUS["refused"].get(event, 0) + 1


def census():
    """This process's served calls (by shape, capped at 32 keys) and refusals by event."""
    with _LOCK:
        return {k: (dict(v) if isinstance(v, dict) else v) for k, v in CENSUS.items()}


def _dt(t, what):
    if t.dtype == torch.float32:
        return L.DT_F32
    if t.dtype == torch.bfloat16:
        return L.DT_BF16
    raise Unsupported("dtype:%s" % what, str(t.dtype))


def pair_bias_attention(q, k, v, pair_bias, key_mask=None, *, gate=None, num_samples=None, num_heads=None, layout="rows", out=None,
                        scale=None, inf=1e9, config=None):
    """See the module docstring.  Returns [S*N, H*D] (layout rows) or [S, N, H*D] (layout shnd), or ``out``."""
    try:
        if not math.isfinite(float(inf)) or (scale is not None and not math.isfinite(float(scale))):
            raise Unsupported("nonfinite:inf_or_scale", "inf and scale must be finite (inf=%r scale=%r)" % (inf, scale))
        if not q.is_cuda:
            raise Unsupported("device:%s" % q.device.type, "the HIP core serves device tensors")
        if layout == "shnd":
            if q.dim() != 4:
                raise Unsupported("rank", "layout shnd wants q/k/v [S,H,N,D], got %s" % (tuple(q.shape),))
            S, H, N, D = (int(x) for x in q.shape)
            NK = int(k.shape[2])
            if num_samples is not None and int(num_samples) != S:
                raise Unsupported("shape:num_samples", "num_samples=%s but q has S=%d" % (num_samples, S))
            if tuple(k.shape) != (S, H, NK, D) or tuple(v.shape) != (S, H, NK, D):
                raise Unsupported("shape:kv", "k / v must be [S,H,NK,D] = %s" % ((S, H, NK, D),))
            q4 = q.permute(0, 2, 1, 3)                   # [S, N, H, D] views, no copy
            k4 = k.permute(0, 2, 1, 3)
            v4 = v.permute(0, 2, 1, 3)
            g4 = None
            if gate is not None:
                g4 = gate if gate.dim() == 4 else gate.reshape(S, N, H, D) if gate.stride(-1) == 1 else None
                if g4 is None or tuple(g4.shape) != (S, N, H, D):
                    raise Unsupported("shape:gate", "layout shnd wants gate [S,N,H*D] or [S,N,H,D]")
            res = out if out is not None else torch.empty((S, N, H * D), dtype=q.dtype, device=q.device)
            if tuple(res.shape) != (S, N, H * D) or res.stride(-1) != 1:
                raise Unsupported("shape:out", "layout shnd wants out [S,N,H*D] with unit column stride")
            o4 = res.as_strided((S, N, H, D), (res.stride(0), res.stride(1), D, 1), res.storage_offset())
        elif layout == "rows":
            if num_samples is None or num_heads is None:
                raise Unsupported("layout:rows_needs_S_H", "layout rows needs num_samples and num_heads")
            S, H = int(num_samples), int(num_heads)
            for name, t in (("q", q), ("k", k), ("v", v)) + ((("gate", gate),) if gate is not None else ()):
                if t.dim() != 2 or t.shape[0] % S or t.shape[1] % H or t.stride(1) != 1:
                    raise Unsupported("shape:%s" % name, "layout rows wants %s 2-D [S*N, H*D] with unit column stride, got %s strides %s"
                                      % (name, tuple(t.shape), tuple(t.stride())))
            N, D = int(q.shape[0]) // S, int(q.shape[1]) // H
            NK = int(k.shape[0]) // S
            if tuple(v.shape) != tuple(k.shape) or int(k.shape[1]) != H * D:
                raise Unsupported("shape:kv", "layout rows wants k / v [S*NK, H*D]")
            if gate is not None and tuple(gate.shape) != (S * N, H * D):
                raise Unsupported("shape:gate", "layout rows wants gate [S*N, H*D] = %s, got %s" % ((S * N, H * D), tuple(gate.shape)))

            def as4(t, n):                               # [S*n, H*D] rows -> [S, n, H, D] view (no copy)
                rs = t.stride(0)
                return t.as_strided((S, n, H, D), (n * rs, rs, D, 1), t.storage_offset())
            q4, k4, v4 = as4(q, N), as4(k, NK), as4(v, NK)
            g4 = None if gate is None else as4(gate, N)
            res = out if out is not None else torch.empty((S * N, H * D), dtype=q.dtype, device=q.device)
            if res.dim() != 2 or tuple(res.shape) != (S * N, H * D) or res.stride(1) != 1:
                raise Unsupported("shape:out", "layout rows wants out [S*N, H*D] with unit column stride, got %s" % (tuple(res.shape),))
            o4 = as4(res, N)
        else:
            raise Unsupported("layout:%s" % layout, "known layouts: " + ", ".join(LAYOUTS))
        if D not in HEAD_DIMS:
            raise Unsupported("head_dim:%d" % D, "served head dims: %s" % (HEAD_DIMS,))
        dt = _dt(q, "q")
        for name, t in (("k", k), ("v", v)) + ((("gate", gate),) if gate is not None else ()) + (("out", res),):
            if t.dtype != q.dtype:
                raise Unsupported("dtype:mix", "%s is %s, q is %s" % (name, t.dtype, q.dtype))
        pb = pair_bias
        while pb.dim() > 4 and int(pb.shape[0]) == 1:
            pb = pb[0]
        if pb.dim() == 3:
            pb = pb.unsqueeze(0)
        if pb.dim() != 4 or int(pb.shape[0]) not in (1, S) or tuple(pb.shape[1:]) != (H, N, NK):
            raise Unsupported("shape:pair_bias", "pair_bias must be [H,N,NK] or [S|1,H,N,NK], got %s" % (tuple(pair_bias.shape),))
        if pb.stride(-1) != 1:
            raise Unsupported("stride:pair_bias", "pair_bias needs a unit key stride")
        bdt = _dt(pb, "pair_bias")
        km, mdt = None, L.DT_U8
        if key_mask is not None:
            km = key_mask
            while km.dim() > 2 and int(km.shape[0]) == 1:
                km = km[0]
            if km.dim() == 1:
                km = km[None, :]
            if km.dim() != 2 or int(km.shape[0]) not in (1, S) or int(km.shape[1]) != NK:
                raise Unsupported("shape:mask", "key_mask must be [NK], [1,NK] or [S,NK], got %s" % (tuple(key_mask.shape),))
            if km.dtype == torch.float32:
                mdt = L.DT_F32
            elif km.dtype in (torch.bool, torch.uint8):
                km = km.view(torch.uint8)
            else:
                km = (km != 0).view(torch.uint8)
        a = L.ApbArgs(abi_version=L.ABI_VERSION, dtype=dt, S=S, N=N, NK=NK, H=H, D=D, q=L.ptr(q4), k=L.ptr(k4), v=L.ptr(v4),
                      gate=L.ptr(g4), bias=L.ptr(pb), bias_dtype=bdt, key_mask=L.ptr(km), mask_dtype=mdt, out=L.ptr(o4),
                      scale=(1.0 / math.sqrt(D)) if scale is None else float(scale))
        a.q_stride[:] = list(q4.stride())
        a.k_stride[:] = list(k4.stride())
        a.v_stride[:] = list(v4.stride())
        a.out_stride[:] = list(o4.stride())
        if g4 is not None:
            a.gate_stride[:] = list(g4.stride())
        bs = list(pb.stride())
        a.bias_stride[:] = [0 if int(pb.shape[0]) == 1 else bs[0], bs[1], bs[2], bs[3]]
        if km is not None:
            a.mask_stride[:] = [0 if int(km.shape[0]) == 1 else km.stride(0), km.stride(1)]
        try:
            L.call("fpf_apb_fwd", a, L.stream_ptr(q.device))
        except L.LibError as e:
            raise Unsupported("lib:%s" % e.kind, e.msg)
    except Unsupported as e:
        _book(e.event)
        raise
    _book(None, "S%dH%dN%dD%d" % (S, H, N, D))
    return res


def pair_bias_producer(z, w_z, ln_w=None, ln_b=None, *, eps=1e-5, dtype=torch.float32, out=None):
    """bias[b, h, i, j] = LayerNorm(z[b, i, j, :]) . w_z[h, :] for bf16 z [B, N, N, 128] (or [N, N, 128]) and w_z [H, 128], H <= 32.
    Returns [B, H, N, N] in ``dtype`` (fp32 | bf16); ``out`` may be a [B, H, N, N] view with unit key stride and any row pitch >= N."""
    z4 = z if z.dim() == 4 else z.unsqueeze(0)
    if z4.dtype != torch.bfloat16 or not z4.is_contiguous():
        raise Unsupported("dtype:z", "the producer reads contiguous bf16 z")
    B, N, _, C = (int(x) for x in z4.shape)
    H = int(w_z.shape[0])
    if C != 128 or tuple(w_z.shape) != (H, C) or not 1 <= H <= 32:
        raise Unsupported("shape:w_z", "w_z [H <= 32, 128] for z [.., 128], got %s" % (tuple(w_z.shape),))
    if out is None:
        out = torch.empty((B, H, N, N), dtype=dtype, device=z.device)
    if tuple(out.shape) != (B, H, N, N) or out.stride(-1) != 1 or out.stride(1) != N * out.stride(2) or out.stride(0) != H * out.stride(1):
        raise Unsupported("shape:out", "out must be [B,H,N,N] with rows of one pitch")
    wz = w_z.to(device=z.device, dtype=torch.bfloat16).contiguous()
    lw = None if ln_w is None else ln_w.to(device=z.device, dtype=torch.float32).contiguous()
    lb = None if ln_b is None else ln_b.to(device=z.device, dtype=torch.float32).contiguous()
    a = L.ApbBiasArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, B=B, N=N, C=C, H=H, z=L.ptr(z4), ln_w=L.ptr(lw), ln_b=L.ptr(lb),
                      eps=float(eps), w_z=L.ptr(wz), bias=L.ptr(out), bias_dtype=_dt(out, "bias"), bias_ld=int(out.stride(2)))
    try:
        L.call("fpf_apb_bias_fwd", a, L.stream_ptr(z.device))
    except L.LibError as e:
        raise Unsupported("lib:%s" % e.kind, e.msg)
    return out


class ApbWeights(object):
    """One AttentionPairBias module's weights on the device (fp32; the bias producer's w_z in bf16): the q|k|v|g projection packed
    as one [4 c_s, c_s] matrix (q's bias in the first c_s entries of a [4 c_s] vector), proj_o, proj_z's LayerNorm and linear."""

    def __init__(self, P, device):
        dev = torch.device(device)
        f = lambda t: t.detach().to(device=dev, dtype=torch.float32).contiguous()     # noqa: E731
        self.H = int(P["H"])
        self.c_s = int(P["w_q"].shape[0])
        self.w_qkvg = torch.cat([f(P["w_q"]), f(P["w_k"]), f(P["w_v"]), f(P["w_g"])], 0).contiguous()
        self.b_qkvg = torch.cat([f(P["b_q"]), torch.zeros(3 * self.c_s, device=dev)], 0)
        self.w_o = f(P["w_o"])
        self.ln_z_w, self.ln_z_b = f(P["ln_z_w"]), f(P["ln_z_b"])
        self.w_z = P["w_z"].detach().to(device=dev, dtype=torch.bfloat16).contiguous()


def attention_pair_bias_module(s_n, z, mask, W, *, bias=None):
    """AttentionPairBias.forward (attentionv2.py:62-111) with k_in = s_n: s_n [B, N, c_s] fp32 (already normalised), z the bf16 pair
    tensor [B, N, N, 128] (or ``bias`` [B, H, N, N] already produced), mask [B, N] token mask.  Returns the update [B, N, c_s] fp32."""
    B, N, CS = (int(x) for x in s_n.shape)
    H = W.H
    proj = torch.addmm(W.b_qkvg, s_n.reshape(B * N, CS), W.w_qkvg.t())              # [B*N, 4 c_s]: q | k | v | g column blocks
    if bias is None:
        bias = pair_bias_producer(z, W.w_z, W.ln_z_w, W.ln_z_b)
    o = torch.empty((B * N, CS), dtype=torch.float32, device=s_n.device)
    for b in range(B):                                                              # one bias plane per batch element
        rows = slice(b * N, (b + 1) * N)
        pair_bias_attention(proj[rows, :CS], proj[rows, CS:2 * CS], proj[rows, 2 * CS:3 * CS], bias[b], None if mask is None else mask[b],
                            gate=proj[rows, 3 * CS:], num_samples=1, num_heads=H, layout="rows", out=o[rows])
    return torch.matmul(o, W.w_o.t()).view(B, N, CS)

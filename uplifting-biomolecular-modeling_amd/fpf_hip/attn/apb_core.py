"""Attention with a pair bias over libfpf_hip (``fpf_apb_fwd``; the producer ``fpf_apb_bias_fwd``): the Pairformer single track's
AttentionPairBias and the token attention of a sample batch sharing one bias.

Serves the face of common/opt_core/opt_core/attn/apb_core.py -- the refusal type with its ``event`` / ``detail`` (:45), the
per-process ``census()`` (:63) and

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
import collections
import math
import threading

import torch

from .. import _lib as L

LAYOUTS = ("rows", "shnd")
HEAD_DIMS = (16, 24, 32, 48, 64)


class Unsupported(Exception):
    """Raised before anything is launched when a call falls outside what the HIP core serves.  ``event`` is the census word
    (``layout:<name>``, ``shape:<operand>``, ``dtype:<operand>``, ``stride:<operand>``, ``head_dim:<n>``, ``device:<type>``,
    ``rank``, ``nonfinite:inf_or_scale``, ``lib:<kind>``); ``detail`` says what was found."""

    def __init__(self, event, detail=""):
        self.event, self.detail = event, detail
        Exception.__init__(self, event + (": " + detail if detail else ""))


class _Ledger(object):
    """Per-process counts of this face's calls: served calls (in all and per problem shape) and refusals per event word.  At most
    SHAPES distinct shapes are named; calls of further shapes are counted under "other"."""
    SHAPES = 32

    def __init__(self):
        self._mu = threading.Lock()
        self.served = 0
        self.refused = collections.Counter()
        self.by_shape = collections.Counter()

    def serve(self, shape):
        with self._mu:
            self.served += 1
            self.by_shape[shape if shape in self.by_shape or len(self.by_shape) < self.SHAPES else "other"] += 1

    def refuse(self, event):
        with self._mu:
            self.refused[event] += 1

    def snapshot(self):
        with self._mu:
            return {"served": self.served, "refused": dict(self.refused), "by_shape": dict(self.by_shape)}


LEDGER = _Ledger()


def census():
    """{"served": n, "refused": {event: n}, "by_shape": {"S..H..N..D..": n}} for this process."""
    return LEDGER.snapshot()


def _require(ok, event, detail=""):
    if not ok:
        raise Unsupported(event, detail)


def _heads_view(t, S, n, H, D):
    """[S*n, H*D] row block (unit column stride, any row stride) -> its [S, n, H, D] view."""
    r = t.stride(0)
    return t.as_strided((S, n, H, D), (n * r, r, D, 1), t.storage_offset())


class _Problem(object):
    """The operands of one call as [S, N|NK, H, D] views plus the result tensor handed back to the caller."""
    __slots__ = ("S", "N", "NK", "H", "D", "q", "k", "v", "gate", "o", "result")


def _rows_problem(q, k, v, gate, out, num_samples, num_heads):
    """Layout "rows": every operand a 2-D row block [S*rows, H*D] with unit column stride, e.g. column slices of one fused
    q|k|v|g projection output."""
    _require(num_samples is not None and num_heads is not None, "layout:rows_needs_S_H", "num_samples and num_heads are required")
    P = _Problem()
    P.S, P.H = int(num_samples), int(num_heads)
    named = [("q", q), ("k", k), ("v", v)] + ([("gate", gate)] if gate is not None else [])
    for name, t in named:
        _require(t.dim() == 2 and t.stride(1) == 1 and t.shape[0] % P.S == 0 and t.shape[1] % P.H == 0, "shape:" + name,
                 "%s is %s with strides %s; a 2-D block of S*rows x H*D with unit column stride is needed"
                 % (name, tuple(t.shape), tuple(t.stride())))
    P.N, P.D = int(q.shape[0]) // P.S, int(q.shape[1]) // P.H
    P.NK = int(k.shape[0]) // P.S
    _require(int(k.shape[1]) == P.H * P.D and tuple(v.shape) == tuple(k.shape), "shape:kv",
             "k %s and v %s must both be [S*NK, %d]" % (tuple(k.shape), tuple(v.shape), P.H * P.D))
    _require(gate is None or tuple(gate.shape) == (P.S * P.N, P.H * P.D), "shape:gate",
             "gate %s, query rows need %s" % (None if gate is None else tuple(gate.shape), (P.S * P.N, P.H * P.D)))
    res = out if out is not None else torch.empty((P.S * P.N, P.H * P.D), dtype=q.dtype, device=q.device)
    _require(res.dim() == 2 and tuple(res.shape) == (P.S * P.N, P.H * P.D) and res.stride(1) == 1, "shape:out",
             "out %s; a [%d, %d] block with unit column stride is needed" % (tuple(res.shape), P.S * P.N, P.H * P.D))
    P.q, P.k, P.v = _heads_view(q, P.S, P.N, P.H, P.D), _heads_view(k, P.S, P.NK, P.H, P.D), _heads_view(v, P.S, P.NK, P.H, P.D)
    P.gate = None if gate is None else _heads_view(gate, P.S, P.N, P.H, P.D)
    P.o, P.result = _heads_view(res, P.S, P.N, P.H, P.D), res
    return P


def _shnd_problem(q, k, v, gate, out, num_samples):
    """Layout "shnd": q, k, v [S, H, rows, D] (innermost stride 1, served through their strides), gate [S, N, H*D] or
    [S, N, H, D]."""
    _require(q.dim() == 4, "rank", "q has shape %s; [S, H, N, D] expected" % (tuple(q.shape),))
    P = _Problem()
    P.S, P.H, P.N, P.D = (int(x) for x in q.shape)
    P.NK = int(k.shape[2]) if k.dim() == 4 else -1
    _require(num_samples is None or int(num_samples) == P.S, "shape:num_samples", "num_samples=%s, q holds %d samples" % (num_samples, P.S))
    _require(tuple(k.shape) == (P.S, P.H, P.NK, P.D) and tuple(v.shape) == tuple(k.shape), "shape:kv",
             "k %s, v %s; both [%d, %d, NK, %d] expected" % (tuple(k.shape), tuple(v.shape), P.S, P.H, P.D))
    P.q, P.k, P.v = (t.permute(0, 2, 1, 3) for t in (q, k, v))          # [S, rows, H, D] views
    P.gate = None
    if gate is not None:
        g4 = None
        if gate.dim() == 3 and tuple(gate.shape) == (P.S, P.N, P.H * P.D) and gate.stride(-1) == 1:
            g4 = gate.as_strided((P.S, P.N, P.H, P.D), (gate.stride(0), gate.stride(1), P.D, 1), gate.storage_offset())
        elif gate.dim() == 4 and tuple(gate.shape) == (P.S, P.N, P.H, P.D) and gate.stride(-1) == 1:
            g4 = gate
        _require(g4 is not None, "shape:gate", "gate %s; [S, N, H*D] or [S, N, H, D] with unit innermost stride expected" % (tuple(gate.shape),))
        P.gate = g4
    res = out if out is not None else torch.empty((P.S, P.N, P.H * P.D), dtype=q.dtype, device=q.device)
    _require(tuple(res.shape) == (P.S, P.N, P.H * P.D) and res.stride(-1) == 1, "shape:out",
             "out %s; [%d, %d, %d] with unit column stride expected" % (tuple(res.shape), P.S, P.N, P.H * P.D))
    P.o = res.as_strided((P.S, P.N, P.H, P.D), (res.stride(0), res.stride(1), P.D, 1), res.storage_offset())
    P.result = res
    return P


def _drop_unit_dims(t, keep):
    """``t`` without leading size-1 dimensions beyond its last ``keep`` ones."""
    while t.dim() > keep and int(t.shape[0]) == 1:
        t = t.squeeze(0)
    return t


def _storage_code(t, what):
    codes = {torch.float32: L.DT_F32, torch.bfloat16: L.DT_BF16}
    _require(t.dtype in codes, "dtype:" + what, "%s is %s; fp32 or bf16 storage is served" % (what, t.dtype))
    return codes[t.dtype]


def pair_bias_attention(q, k, v, pair_bias, key_mask=None, *, gate=None, num_samples=None, num_heads=None, layout="rows", out=None,
                        scale=None, inf=1e9, config=None):
    """See the module docstring.  Returns [S*N, H*D] (layout rows) or [S, N, H*D] (layout shnd), or ``out``."""
    try:
        _require(math.isfinite(float(inf)) and (scale is None or math.isfinite(float(scale))), "nonfinite:inf_or_scale",
                 "a masked key is dropped by name, so inf and scale must be finite numbers (inf=%r, scale=%r)" % (inf, scale))
        _require(q.is_cuda, "device:%s" % q.device.type, "q is on %s; the HIP core reads device memory" % q.device)
        if layout == "rows":
            P = _rows_problem(q, k, v, gate, out, num_samples, num_heads)
        elif layout == "shnd":
            P = _shnd_problem(q, k, v, gate, out, num_samples)
        else:
            raise Unsupported("layout:%s" % (layout,), "served layouts: %s" % (", ".join(LAYOUTS),))
        _require(P.D in HEAD_DIMS, "head_dim:%d" % P.D, "head dims with a compiled kernel: %s" % (HEAD_DIMS,))
        dt = _storage_code(q, "q")
        for name, t in (("k", k), ("v", v), ("gate", gate), ("out", P.result)):
            _require(t is None or t.dtype == q.dtype, "dtype:mix", "%s is %s while q is %s" % (name, None if t is None else t.dtype, q.dtype))
        pb = _drop_unit_dims(pair_bias, 4)
        pb = pb.unsqueeze(0) if pb.dim() == 3 else pb
        _require(pb.dim() == 4 and int(pb.shape[0]) in (1, P.S) and tuple(pb.shape[1:]) == (P.H, P.N, P.NK), "shape:pair_bias",
                 "pair_bias %s; [H, N, NK] or [1 | S, H, N, NK] with H=%d N=%d NK=%d expected" % (tuple(pair_bias.shape), P.H, P.N, P.NK))
        _require(pb.stride(-1) == 1, "stride:pair_bias", "the key axis of pair_bias must have unit stride")
        bias_code = _storage_code(pb, "pair_bias")
        km, mask_code = None, L.DT_U8
        if key_mask is not None:
            km = _drop_unit_dims(key_mask, 2)
            km = km.unsqueeze(0) if km.dim() == 1 else km
            _require(km.dim() == 2 and int(km.shape[0]) in (1, P.S) and int(km.shape[1]) == P.NK, "shape:mask",
                     "key_mask %s; [NK], [1, NK] or [S, NK] with NK=%d expected" % (tuple(key_mask.shape), P.NK))
            if km.dtype == torch.float32:
                mask_code = L.DT_F32
            else:
                km = (km if km.dtype in (torch.bool, torch.uint8) else km != 0).view(torch.uint8)
        a = L.ApbArgs(abi_version=L.ABI_VERSION, dtype=dt, S=P.S, N=P.N, NK=P.NK, H=P.H, D=P.D, q=L.ptr(P.q), k=L.ptr(P.k),
                      v=L.ptr(P.v), gate=L.ptr(P.gate), bias=L.ptr(pb), bias_dtype=bias_code, key_mask=L.ptr(km), mask_dtype=mask_code,
                      out=L.ptr(P.o), scale=(1.0 / math.sqrt(P.D)) if scale is None else float(scale))
        for field, t in (("q_stride", P.q), ("k_stride", P.k), ("v_stride", P.v), ("out_stride", P.o), ("gate_stride", P.gate)):
            if t is not None:
                getattr(a, field)[:] = list(t.stride())
        shared = int(pb.shape[0]) == 1
        a.bias_stride[:] = [0 if shared else pb.stride(0)] + list(pb.stride()[1:])
        if km is not None:
            a.mask_stride[:] = [0 if int(km.shape[0]) == 1 else km.stride(0), km.stride(1)]
        try:
            L.call("fpf_apb_fwd", a, L.stream_ptr(q.device))
        except L.LibError as e:
            raise Unsupported("lib:%s" % e.kind, e.msg)
    except Unsupported as e:
        LEDGER.refuse(e.event)
        raise
    LEDGER.serve("S%dH%dN%dD%d" % (P.S, P.H, P.N, P.D))
    return P.result


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
                      eps=float(eps), w_z=L.ptr(wz), bias=L.ptr(out), bias_dtype=_storage_code(out, "bias"), bias_ld=int(out.stride(2)))
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

"""The stock PyTorch statements of the pair-stack hot path, restated on the CPU -- TEST INFRASTRUCTURE ONLY.

Every function evaluates in ``dtype`` (float64 by default; float32 for the fp32 yardstick the BASELINE tolerances are stated
against) on CPU tensors and returns a tensor of that dtype.  The pair-block statements also accept device tensors (inputs and
parameters on one device; the results are allocated there): the N = 768 stack checks evaluate the same fp32 statements on the
GPU, where the CPU would take minutes per block.  They are the checker of the HIP path and the timed CPU baseline of
``bench.py``; nothing in the product imports them.

Reference statements followed (paths under the reference tree):
    layer_norm            torch.nn.LayerNorm as used by every module below (biased variance, eps inside the sqrt)
    triangle_attention_op common/opt_core/opt_core/kernels/triattn/__init__.py:3-8 (op contract), :1202-1220 (``reference``:
                          -inf at masked keys, a fully-masked row is uniform over all keys)
    tri_attn              boltz2/stock/src/boltz/model/layers/triangular_attention/attention.py:108-179 and
                          primitives.py:126-156 (LayerNorm), :159-196 (softmax, _attention), :265-366 (Attention: q/sqrt(c),
                          sigmoid gate, linear_o); the 1e9*(mask-1) additive mask of attention.py:149
    trimul                boltz2/stock/src/boltz/model/layers/triangular_mult.py:73-124 (outgoing), :161-212 (incoming);
                          ten-tensor vocabulary of common/opt_core/opt_core/kernels/trimul/__init__.py:3-11, :1946-1979
    transition            boltz2/stock/src/boltz/model/layers/transition.py:47-78;
                          common/opt_core/opt_core/kernels/transition/__init__.py:5-10, :1022-1032 (mask, residual)
    pair_block            boltz2/stock/src/boltz/model/layers/pairformer.py:75-102 (order and residual adds; dropout = 1 in eval)
    triatt_prologue /     common/opt_core/opt_core/attn/pair_fused.py:1136-1233 (q,k,v [B,I,H,J,D], g [B,I,J,HD] pre-sigmoid,
    triatt_epilogue       bias [B,1,H,I,J] in the attention frame) and :1416-1498 (u = (sigmoid(g) o) W_o^T, residual into z,
                          transposed scatter for the ending node)
    pair_bias_attention_op common/opt_core/opt_core/attn/apb_core.py:1-12 (op contract: shared or per-sample bias, key mask,
                          sigmoid gate; a sample whose keys are all masked is uniform over all keys)
    pair_bias             boltz2/stock/src/boltz/model/layers/attentionv2.py:53-58 (proj_z: LayerNorm(c_z) -> Linear(c_z, H) ->
                          heads first)
    attention_pair_bias   attentionv2.py:62-111 (AttentionPairBias forward, compute_pair_bias=True: q with bias, k / v / g
                          without, fp32 softmax with the additive (1 - mask) * -inf key mask, sigmoid gate, proj_o)
    single_track /        boltz2/stock/src/boltz/model/layers/pairformer.py:104-111 (pre_norm_s, s += attention(s_n, z, mask,
    pairformer_layer      k_in = s_n), s += transition_s(s); post norm = identity) after the pair stack :75-102
"""
import math

import torch

__all__ = ["layer_norm", "triangle_attention_op", "tri_attn", "triatt_prologue", "triatt_epilogue", "trimul", "trimul_rows",
           "trimul_autocast", "tri_attn_autocast", "transition_autocast", "pair_block_autocast",
           "tri_attn_rows", "transition", "pair_block", "make_block_params", "block_flops", "pair_bias_attention_op", "pair_bias",
           "attention_pair_bias", "single_track", "pairformer_layer", "make_single_params", "single_flops"]


def layer_norm(x, w=None, b=None, eps=1e-5):
    """(x - mean) / sqrt(var + eps) * w + b over the last axis, biased variance, evaluated in x's dtype.
    Pinned by: torch.nn.functional.layer_norm (library routine), constant rows -> b (tests/test_oracle.py)."""
    mu = x.mean(dim=-1, keepdim=True)
    xc = x - mu
    var = (xc * xc).mean(dim=-1, keepdim=True)
    y = xc / torch.sqrt(var + eps)
    if w is not None:
        y = y * w.to(x.dtype)
    if b is not None:
        y = y + b.to(x.dtype)
    return y


def triangle_attention_op(q, k, v, bias, mask=None, scale=None, dtype=torch.float64, rows_per_step=32):
    """out[b,n,h,i,:] = softmax_j(scale q.k + bias[b,0,h,i,j], -inf where mask[b,n,0,0,j] is False) @ v[b,n,h,j,:].
    q/k/v [B,N,H,S,D], bias [B,1,H,S,S], mask [B,N,1,1,S] bool (or None).  A fully-masked row is the uniform mean of v over all
    keys (triattn/__init__.py:1202-1220).
    Pinned by: the reference's fp64 rows (tests/golden/triattn_*), S = 1 -> v, key-permutation equivariance, bias row-shift
    invariance, brute force (tests/test_oracle.py)."""
    B, N, H, S, D = q.shape
    sc = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    out = torch.empty(B, N, H, S, D, dtype=dtype, device=q.device)
    bias_ = bias.to(dtype)
    for n0 in range(0, N, rows_per_step):
        n1 = min(N, n0 + rows_per_step)
        s = torch.matmul(q[:, n0:n1].to(dtype), k[:, n0:n1].to(dtype).transpose(-1, -2)) * sc + bias_
        if mask is not None:
            keep = mask[:, n0:n1].reshape(B, n1 - n0, 1, 1, S).to(torch.bool)
            dead = ~keep.any(dim=-1, keepdim=True)
            s = torch.where(keep | dead, s, torch.full_like(s, float("-inf")))
            s = torch.where(dead.expand_as(s), torch.zeros_like(s), s)
        out[:, n0:n1] = torch.matmul(torch.softmax(s, dim=-1), v[:, n0:n1].to(dtype))
    return out


def _as4(z):
    return (z, False) if z.dim() == 4 else (z.unsqueeze(0), True)


def tri_attn(z, P, mask=None, *, ending=False, dtype=torch.float64, rows_per_step=64, inf=1e9, x_ln=None):
    """Stock TriangleAttention{Starting,Ending}Node forward -> the update in z's frame ([B,N,N,C] or [N,N,C]).
    P: dict ln_w, ln_b [C], w_q, w_k, w_v, w_g [H*D, C], w_b [H, C], w_o [C, H*D], plus ints H, D; optional b_g [H*D] (linear_g
    bias) and b_o [C] (linear_o bias), the Linear biases of primitives.py:259-270 where a kit's module carries them.
    The ending node transposes z (and the mask) in and the update out (attention.py:140-142, :175-176).  ``x_ln``: the caller's
    own LayerNorm output in the attention frame, used in place of LN(x) (pair_fused.py:1151-1160, ln="stock").
    Pinned by: scalar loops over the published equations (starting and ending node each in its own index form), ending(z) ==
    starting(z^T)^T, the op form (triangle_attention_op) on the same projections, and the BASELINE config-1 block
    (tests/test_oracle.py)."""
    z4, sq = _as4(z)
    B, N, _, C = z4.shape
    H, D = int(P["H"]), int(P["D"])
    x = z4.to(dtype)
    m = torch.ones(B, N, N, dtype=dtype, device=z4.device) if mask is None else (mask if mask.dim() == 3 else mask.unsqueeze(0)).to(dtype)
    if ending:
        x = x.transpose(1, 2)
        m = m.transpose(1, 2)
    x = layer_norm(x, P["ln_w"], P["ln_b"], 1e-5) if x_ln is None else _as4(x_ln)[0].to(dtype)
    wq, wk, wv, wg = (P[n].to(dtype) for n in ("w_q", "w_k", "w_v", "w_g"))
    wb, wo = P["w_b"].to(dtype), P["w_o"].to(dtype)
    bg = None if P.get("b_g") is None else P["b_g"].to(dtype)
    bo = None if P.get("b_o") is None else P["b_o"].to(dtype)
    tri_bias = torch.matmul(x, wb.t()).permute(0, 3, 1, 2).unsqueeze(1)          # [B, 1, H, I, J]
    out = torch.empty(B, N, N, wo.shape[0], dtype=dtype, device=x.device)
    for i0 in range(0, N, rows_per_step):
        i1 = min(N, i0 + rows_per_step)
        xi = x[:, i0:i1]                                                            # [B, r, J, C]
        mask_bias = (inf * (m[:, i0:i1] - 1.0))[:, :, None, None, :]                # [B, r, 1, 1, J]
        q = torch.matmul(xi, wq.t()).view(B, i1 - i0, N, H, D).transpose(-2, -3) / math.sqrt(D)
        kk = torch.matmul(xi, wk.t()).view(B, i1 - i0, N, H, D).transpose(-2, -3)
        vv = torch.matmul(xi, wv.t()).view(B, i1 - i0, N, H, D).transpose(-2, -3)
        a = torch.matmul(q, kk.transpose(-1, -2)) + mask_bias + tri_bias            # [B, r, H, J, J]
        a = torch.softmax(a, dim=-1)
        o = torch.matmul(a, vv).transpose(-2, -3)                                   # [B, r, J, H, D]
        gl = torch.matmul(xi, wg.t())
        g = torch.sigmoid(gl if bg is None else gl + bg).view(B, i1 - i0, N, H, D)
        u = torch.matmul((o * g).reshape(B, i1 - i0, N, H * D), wo.t())
        out[:, i0:i1] = u if bo is None else u + bo
    if ending:
        out = out.transpose(1, 2)
    return out[0] if sq else out


def triatt_prologue(z, P, *, ending=False, dtype=torch.float64):
    """The block prologue's tensors in the attention frame x = z (or z^T): q, k, v [B,I,H,J,D], g [B,I,J,H*D] (pre-sigmoid),
    bias [B,1,H,I,J] -- unrounded (pair_fused.py:1136-1233 states the same tensors with bf16 rounding points).
    Pinned by: tri_attn == epilogue(op(prologue)) (tests/test_oracle.py)."""
    z4, _ = _as4(z)
    B, N, _, C = z4.shape
    H, D = int(P["H"]), int(P["D"])
    x = z4.to(dtype)
    if ending:
        x = x.transpose(1, 2)
    x = layer_norm(x, P["ln_w"], P["ln_b"], 1e-5)

    def heads(w):
        return torch.matmul(x, w.to(dtype).t()).view(B, N, N, H, D).permute(0, 1, 3, 2, 4)
    q, k, v = heads(P["w_q"]), heads(P["w_k"]), heads(P["w_v"])
    g = torch.matmul(x, P["w_g"].to(dtype).t())
    if P.get("b_g") is not None:
        g = g + P["b_g"].to(dtype)
    bias = torch.matmul(x, P["w_b"].to(dtype).t()).permute(0, 3, 1, 2).unsqueeze(1)
    return q, k, v, g, bias


def triatt_epilogue(o, g, P, *, dtype=torch.float64):
    """u [B,I,J,C_out] = (sigmoid(g) * o) @ w_o^T (+ b_o) in the attention frame; o [B,I,H,J,D], g [B,I,J,H*D] (b_g already in)."""
    B, I, H, J, D = o.shape
    ot = o.to(dtype).permute(0, 1, 3, 2, 4).reshape(B, I, J, H * D)
    u = torch.matmul(torch.sigmoid(g.to(dtype)) * ot, P["w_o"].to(dtype).t())
    return u if P.get("b_o") is None else u + P["b_o"].to(dtype)


def trimul(z, mask=None, *, direction, weights, residual=False, dtype=torch.float64, eps=1e-5):
    """Stock TriangleMultiplication{Outgoing,Incoming} in the ten-tensor vocabulary:
        x = LN_in(z); a = mask * sigmoid(x W_ag^T) * (x W_ap^T); b likewise;
        X[i,j] = sum_k a[i,k] b[j,k] (outgoing) | sum_k a[k,i] b[k,j] (incoming);
        update = sigmoid(x W_og^T) * (LN_out(X) W_o^T); z + update when residual.
    z [B,N,N,c_z] or [N,N,c_z]; mask [B,N,N] / [N,N] 0/1 or None.
    Pinned by: the reference's closed-form vectors (input SHA-256 + H100 witness outputs within their recorded fp64 error),
    incoming(z) == outgoing(z^T)^T, all-zero mask -> update = sigmoid(x W_og^T) (ln_out_b W_o^T) (tests/test_oracle.py)."""
    z4, sq = _as4(z)
    w = {k_: v_.to(dtype) for k_, v_ in weights.items() if hasattr(v_, "to")}
    x = layer_norm(z4.to(dtype), w["ln_in_w"], w["ln_in_b"], eps)
    m = None
    if mask is not None:
        m = (mask if mask.dim() == 3 else mask.unsqueeze(0)).to(dtype).unsqueeze(-1)
    a = torch.sigmoid(torch.matmul(x, w["w_ag"].t())) * torch.matmul(x, w["w_ap"].t())
    b = torch.sigmoid(torch.matmul(x, w["w_bg"].t())) * torch.matmul(x, w["w_bp"].t())
    if m is not None:
        a = a * m
        b = b * m
    if direction in ("outgoing", "out"):
        X = torch.einsum("bikd,bjkd->bijd", a, b)
    elif direction in ("incoming", "in"):
        X = torch.einsum("bkid,bkjd->bijd", a, b)
    else:
        raise ValueError(direction)
    upd = torch.sigmoid(torch.matmul(x, w["w_og"].t())) * torch.matmul(layer_norm(X, w["ln_out_w"], w["ln_out_b"], eps), w["w_o"].t())
    out = z4.to(dtype) + upd if residual else upd
    return out[0] if sq else out


def trimul_rows(z, mask, rows, *, direction, weights, dtype=torch.float32, eps=1e-5):
    """Rows ``rows`` of ``trimul``'s update (no residual) for one pair tensor z [N, N, c_z]: the statement above with a computed
    only for the rows (outgoing) / columns (incoming) those output rows read, so that sampled rows of an N = 2048 problem fit a
    CPU check.  Pinned by: equality with ``trimul(...)[rows]`` (tests/test_oracle.py)."""
    w = {k_: v_.to(dtype) for k_, v_ in weights.items() if hasattr(v_, "to")}
    x = layer_norm(z.to(dtype), w["ln_in_w"], w["ln_in_b"], eps)
    m = torch.ones(z.shape[0], z.shape[1], 1, dtype=dtype) if mask is None else mask.to(dtype).unsqueeze(-1)
    idx = torch.as_tensor(rows, dtype=torch.long)
    b = torch.sigmoid(torch.matmul(x, w["w_bg"].t())) * torch.matmul(x, w["w_bp"].t()) * m
    if direction in ("outgoing", "out"):
        xa, ma = x[idx], m[idx]                                                      # [R, N(k), C]
        a = torch.sigmoid(torch.matmul(xa, w["w_ag"].t())) * torch.matmul(xa, w["w_ap"].t()) * ma
        X = torch.einsum("rkd,jkd->rjd", a, b)
    elif direction in ("incoming", "in"):
        xa, ma = x[:, idx], m[:, idx]                                                # [N(k), R, C]
        a = torch.sigmoid(torch.matmul(xa, w["w_ag"].t())) * torch.matmul(xa, w["w_ap"].t()) * ma
        X = torch.einsum("krd,kjd->rjd", a, b)
    else:
        raise ValueError(direction)
    xr = x[idx]
    return torch.sigmoid(torch.matmul(xr, w["w_og"].t())) * torch.matmul(layer_norm(X, w["ln_out_w"], w["ln_out_b"], eps), w["w_o"].t())


def tri_attn_rows(z, P, mask, rows, *, ending=False, dtype=torch.float32):
    """Attention-frame rows ``rows`` of the triangle-attention update for one pair tensor z [N, N, C] (x = z, or z^T for the ending
    node): the full bias from every pixel, then the op (-inf mask; a fully masked row is the uniform mean) and the gated output
    projection for those rows only.  Row i of the result is z row i (starting) / z column i (ending) of the update.  Pinned by:
    equality with ``triatt_epilogue(triangle_attention_op(triatt_prologue(...)))`` restricted to the rows (tests/test_oracle.py)."""
    H, D = int(P["H"]), int(P["D"])
    x = z.to(dtype)
    m = torch.ones(z.shape[0], z.shape[1], dtype=torch.bool) if mask is None else mask != 0
    if ending:
        x = x.transpose(0, 1)
        m = m.transpose(0, 1)
    xl = layer_norm(x, P["ln_w"], P["ln_b"], 1e-5)
    N = xl.shape[0]
    idx = torch.as_tensor(rows, dtype=torch.long)
    bias = torch.matmul(xl, P["w_b"].to(dtype).t()).permute(2, 0, 1).unsqueeze(0).unsqueeze(0)       # [1, 1, H, N, N]
    xr = xl[idx]                                                                                      # [R, N, C]

    def heads(wn):
        return torch.matmul(xr, P[wn].to(dtype).t()).view(len(idx), N, H, D).permute(0, 2, 1, 3).unsqueeze(0)
    o = triangle_attention_op(heads("w_q"), heads("w_k"), heads("w_v"), bias, m[idx][None, :, None, None, :], dtype=dtype)
    g = torch.matmul(xr, P["w_g"].to(dtype).t())
    if P.get("b_g") is not None:
        g = g + P["b_g"].to(dtype)
    return triatt_epilogue(o, g.unsqueeze(0), P, dtype=dtype)[0]


def transition(x, w_a, w_b, w_o, ln_w=None, ln_b=None, *, eps=1e-5, mask=None, residual=False, dtype=torch.float64, x_ln=None):
    """y = W_o(silu(W_a n) * (W_b n)), n = LayerNorm(x) (or the caller's own ``x_ln``: pair_fused.py:1089-1094, ln="stock"); optional
    row mask (y * mask) and residual (x + y).
    Pinned by: the reference's H100 stock bytes at c = 256 (tests/golden/transition_*), W_o = 0 -> identity residual, row
    independence (tests/test_oracle.py)."""
    xx = x.to(dtype)
    n = layer_norm(xx, ln_w, ln_b, eps) if x_ln is None else x_ln.to(dtype)
    a = torch.matmul(n, w_a.to(dtype).t())
    h = a * torch.sigmoid(a) * torch.matmul(n, w_b.to(dtype).t())
    y = torch.matmul(h, w_o.to(dtype).t())
    if mask is not None:
        y = y * mask.reshape(y.shape[:-1]).to(dtype)[..., None]
    return xx + y if residual else y


def pair_block(z, mask, params, *, dtype=torch.float64):
    """One Pairformer layer's pair stack (pairformer.py:75-102, eval): z += trimul_out; z += trimul_in; z += tri_att_start;
    z += tri_att_end; z += transition_z.  ``params`` from :func:`make_block_params`."""
    z = z.to(dtype)
    z = z + trimul(z, mask, direction="outgoing", weights=params["tmo"], dtype=dtype)
    z = z + trimul(z, mask, direction="incoming", weights=params["tmi"], dtype=dtype)
    z = z + tri_attn(z, params["tas"], mask, ending=False, dtype=dtype)
    z = z + tri_attn(z, params["tae"], mask, ending=True, dtype=dtype)
    t = params["tr"]
    z = z + transition(z, t["w_a"], t["w_b"], t["w_o"], t["ln_w"], t["ln_b"], dtype=dtype)
    return z


# ------------------------------------------------------------------------------------------------ the bf16-autocast statement
# The stock modules run under torch.autocast(bfloat16) in the reference's fast paths; the reference admits a bf16 kernel when its
# error vs an fp64 statement is at most 1.25x (rms) / 2.5x (max-abs) THIS statement's own error (SAME_CLASS,
# common/opt_core/opt_core/kernels/fpf_trimul_v4/generic.py:42-43).  Restated here with autocast's rounding points made explicit
# (fp32 arithmetic, bf16 rounding where autocast stores bf16): Linear = bf16 operands, fp32 accumulation, bf16 output; LayerNorm
# runs in fp32 (autocast's fp32 list) and returns fp32; elementwise ops on bf16 tensors return bf16; an in-place add into a bf16
# tensor rounds to bf16; a bf16 * fp32 product promotes to fp32; the residual stream z stays fp32 (pairformer.py:75-102).

def _bf(t):
    return t.to(torch.bfloat16).to(torch.float32)


def _lin_ac(x, w, rnd=_bf):
    """autocast Linear / matmul: bf16 operands, fp32 accumulation, bf16 result."""
    return rnd(torch.matmul(rnd(x), rnd(w).t()))


def trimul_autocast(z, mask, *, direction, weights, eps=1e-5, rnd=_bf):
    """TriangleMultiplication{Outgoing,Incoming}.forward under bf16 autocast (triangular_mult.py:110-124 / :198-212): x = LN_in(z)
    fp32; p_in(x), g_in(x) bf16, sigmoid and product bf16; * mask promotes to fp32 (exact); the einsum runs as an autocast bmm
    (bf16 operands, fp32 accumulation, bf16 result); LN_out fp32; p_out, g_out bf16; sigmoid and product bf16."""
    w = {k_: v_.to(torch.float32) for k_, v_ in weights.items() if hasattr(v_, "to")}
    z4, sq = _as4(z)
    x = layer_norm(z4.to(torch.float32), w["ln_in_w"], w["ln_in_b"], eps)
    a = rnd(_lin_ac(x, w["w_ap"], rnd) * rnd(torch.sigmoid(_lin_ac(x, w["w_ag"], rnd))))
    b = rnd(_lin_ac(x, w["w_bp"], rnd) * rnd(torch.sigmoid(_lin_ac(x, w["w_bg"], rnd))))
    if mask is not None:
        m = (mask if mask.dim() == 3 else mask.unsqueeze(0)).to(torch.float32).unsqueeze(-1)
        a, b = a * m, b * m
    if direction in ("outgoing", "out"):
        X = torch.einsum("bikd,bjkd->bijd", a, b)
    else:
        X = torch.einsum("bkid,bkjd->bijd", a, b)
    X = rnd(X)
    out = rnd(_lin_ac(layer_norm(X, w["ln_out_w"], w["ln_out_b"], eps), w["w_o"], rnd) * rnd(torch.sigmoid(_lin_ac(x, w["w_og"], rnd))))
    return out[0] if sq else out


def tri_attn_autocast(z, P, mask=None, *, ending=False, inf=1e9, rows_per_step=64, rnd=_bf):
    """TriangleAttention.forward under bf16 autocast (attention.py:140-176, primitives.py:176-196, :265-366): x = LN(x) fp32;
    triangle_bias = linear(x) bf16; q, k, v bf16, q / sqrt(c) bf16; a = q k^T bf16; a += mask_bias then a += triangle_bias, each
    rounded to bf16 in place; softmax in bf16 (softmax_no_cast); a v bf16; g = sigmoid(linear_g) bf16; o * g bf16; linear_o bf16."""
    z4, sq = _as4(z)
    B, N, _, C = z4.shape
    H, D = int(P["H"]), int(P["D"])
    x = z4.to(torch.float32)
    m = torch.ones(B, N, N, device=z4.device) if mask is None else (mask if mask.dim() == 3 else mask.unsqueeze(0)).to(torch.float32)
    if ending:
        x, m = x.transpose(1, 2), m.transpose(1, 2)
    x = layer_norm(x, P["ln_w"], P["ln_b"], 1e-5)
    tri_bias = _lin_ac(x, P["w_b"], rnd).permute(0, 3, 1, 2).unsqueeze(1)            # [B, 1, H, I, J]
    out = torch.empty(B, N, N, P["w_o"].shape[0], device=z4.device)
    for i0 in range(0, N, rows_per_step):
        i1 = min(N, i0 + rows_per_step)
        xi = x[:, i0:i1]
        r = i1 - i0

        def heads(w):
            return _lin_ac(xi, w, rnd).view(B, r, N, H, D).transpose(-2, -3)
        q = rnd(heads(P["w_q"]) / math.sqrt(D))
        k, v = heads(P["w_k"]), heads(P["w_v"])
        a = rnd(torch.matmul(q, k.transpose(-1, -2)))
        a = rnd(a + (inf * (m[:, i0:i1] - 1.0))[:, :, None, None, :])
        a = rnd(a + tri_bias)
        a = rnd(torch.softmax(a, dim=-1))
        o = rnd(torch.matmul(a, v)).transpose(-2, -3)                                    # [B, r, J, H, D]
        gl = _lin_ac(xi, P["w_g"], rnd)
        if P.get("b_g") is not None:
            gl = rnd(gl + rnd(P["b_g"]))
        g = rnd(torch.sigmoid(gl)).view(B, r, N, H, D)
        u = _lin_ac(rnd(o * g).reshape(B, r, N, H * D), P["w_o"], rnd)
        out[:, i0:i1] = u if P.get("b_o") is None else rnd(u + rnd(P["b_o"]))
    if ending:
        out = out.transpose(1, 2)
    return out[0] if sq else out


def transition_autocast(x, w_a, w_b, w_o, ln_w=None, ln_b=None, *, eps=1e-5, rnd=_bf):
    """Transition.forward under bf16 autocast (transition.py:63-66): LN fp32; fc1, fc2 bf16; silu bf16; product bf16; fc3 bf16."""
    n = layer_norm(x.to(torch.float32), ln_w, ln_b, eps)
    return _lin_ac(rnd(rnd(torch.nn.functional.silu(_lin_ac(n, w_a, rnd))) * _lin_ac(n, w_b, rnd)), w_o, rnd)


def pair_block_autocast(z, mask, params, *, rnd=_bf):
    """The pair stack of pairformer.py:75-102 under bf16 autocast: every site's statement above, the residual stream fp32.
    ``rnd`` = the identity turns every rounding point off (then this is the fp32 statement ``pair_block``: its pin)."""
    z = z.to(torch.float32)
    z = z + trimul_autocast(z, mask, direction="outgoing", weights=params["tmo"], rnd=rnd)
    z = z + trimul_autocast(z, mask, direction="incoming", weights=params["tmi"], rnd=rnd)
    z = z + tri_attn_autocast(z, params["tas"], mask, ending=False, rnd=rnd)
    z = z + tri_attn_autocast(z, params["tae"], mask, ending=True, rnd=rnd)
    t = params["tr"]
    return z + transition_autocast(z, t["w_a"], t["w_b"], t["w_o"], t["ln_w"], t["ln_b"], rnd=rnd)


def make_block_params(c_z=128, heads=4, head_dim=32, factor=4, seed=0):
    """BASELINE config-1 weights: N(0, 1/fan_in) from torch.Generator('cpu').manual_seed(seed), drawn in module order
    (trimul out, trimul in, tri-att start, tri-att end, transition) and parameter order within a module; LayerNorm weight 1,
    bias 0.  fp32 CPU tensors.  The boltz p_in / g_in halves map onto the ten-tensor vocabulary as
    boltz2/opt/boltz2_opt/trimul.py:64-68 does (first half -> a, second half -> b)."""
    g = torch.Generator("cpu").manual_seed(seed)
    C, H, D = c_z, heads, head_dim
    HD = H * D

    def lin(o, i):
        return torch.randn(o, i, generator=g, dtype=torch.float32) / math.sqrt(i)

    def tm():
        p_in, g_in = lin(2 * C, C), lin(2 * C, C)
        p_out, g_out = lin(C, C), lin(C, C)
        return {"ln_in_w": torch.ones(C), "ln_in_b": torch.zeros(C), "w_ap": p_in[:C].contiguous(), "w_bp": p_in[C:].contiguous(),
                "w_ag": g_in[:C].contiguous(), "w_bg": g_in[C:].contiguous(), "ln_out_w": torch.ones(C), "ln_out_b": torch.zeros(C),
                "w_o": p_out, "w_og": g_out}

    def ta():
        w_b = lin(H, C)                                             # TriangleAttention.linear (c_in -> heads), then mha q, k, v, o, g
        w_q, w_k, w_v = lin(HD, C), lin(HD, C), lin(HD, C)
        w_o = lin(C, HD)
        w_g = lin(HD, C)
        return {"ln_w": torch.ones(C), "ln_b": torch.zeros(C), "w_q": w_q, "w_k": w_k, "w_v": w_v, "w_g": w_g, "w_b": w_b,
                "w_o": w_o, "H": H, "D": D}

    params = {"tmo": tm(), "tmi": tm(), "tas": ta(), "tae": ta()}
    hid = factor * C
    params["tr"] = {"ln_w": torch.ones(C), "ln_b": torch.zeros(C), "w_a": lin(hid, C), "w_b": lin(hid, C), "w_o": lin(C, hid)}
    return params


def block_flops(n, c_z=128, c_h=128, heads=4, head_dim=32, factor=4):
    """Algorithmic FLOPs (2 per multiply-add) of one pair block, per op:
    trimul (one direction) 2N^2(4 c_z c_h + c_z^2 + c_h c_z) + 2N^3 c_h; tri-att (one node) 2N^2 c_z(4HD + H) + 4N^3 HD
    + 2N^2 HD c_z; transition 2N^2 (3 factor c_z^2)."""
    N = n
    HD = heads * head_dim
    tm = 2 * N * N * (4 * c_z * c_h + c_z * c_z + c_h * c_z) + 2 * N ** 3 * c_h
    ta_pro = 2 * N * N * c_z * (4 * HD + heads)
    ta_core = 4 * N ** 3 * HD
    ta_epi = 2 * N * N * HD * c_z
    tr = 2 * N * N * 3 * factor * c_z * c_z
    return {"trimul": tm, "triatt": ta_pro + ta_core + ta_epi, "triatt_core": ta_core, "triatt_prologue": ta_pro,
            "triatt_epilogue": ta_epi, "transition": tr, "block": 2 * tm + 2 * (ta_pro + ta_core + ta_epi) + tr}


# ---------------------------------------------------------------------------------------------------------------- single track
def pair_bias_attention_op(q, k, v, bias, key_mask=None, gate=None, scale=None, dtype=torch.float64):
    """out[s,n,h,:] = sigmoid(gate[s,n,h,:]) * softmax_m(scale q[s,n,h].k[s,m,h] + bias[s|0,h,n,m], masked keys excluded) @ v[s,m,h].
    q [S,N,H,D], k / v [S,NK,H,D], bias [H,N,NK] or [SB,H,N,NK] (SB in {1, S}), key_mask [NK] / [S|1,NK] (nonzero = attend) or None,
    gate [S,N,H,D] or None.  A sample whose keys are all masked attends uniformly to every key (apb_core.py:1-12).
    Pinned by: brute-force scalar loops, key-permutation equivariance, a shared bias equals the per-sample copy, S = 1 with one key
    -> v (tests/test_oracle.py)."""
    S, N, H, D = q.shape
    NK = k.shape[1]
    sc = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    b = bias.to(dtype)
    if b.dim() == 3:
        b = b.unsqueeze(0)
    logits = torch.einsum("snhd,smhd->shnm", q.to(dtype), k.to(dtype)) * sc + b          # [S, H, N, NK]
    if key_mask is not None:
        km = key_mask.reshape(-1, NK).to(torch.bool)
        km = km.expand(S, NK)
        dead = ~km.any(dim=-1)                                                          # [S]
        keep = km | dead[:, None]
        logits = logits.masked_fill(~keep[:, None, None, :], float("-inf"))
        logits = torch.where(dead[:, None, None, None], torch.zeros_like(logits), logits)
    p = torch.softmax(logits, dim=-1)
    o = torch.einsum("shnm,smhd->snhd", p, v.to(dtype))
    if gate is not None:
        o = o * torch.sigmoid(gate.to(dtype))
    return o


def pair_bias(z, ln_w, ln_b, w_z, *, eps=1e-5, dtype=torch.float64):
    """bias[b, h, i, j] = LayerNorm(z[b, i, j, :]) . w_z[h, :] (attentionv2.py:53-58).  z [B,N,N,C] -> [B,H,N,N]."""
    zz = _as4(z)[0].to(dtype)
    return torch.matmul(layer_norm(zz, ln_w, ln_b, eps), w_z.to(dtype).t()).permute(0, 3, 1, 2)


def attention_pair_bias(s, z, mask, P, *, dtype=torch.float64, inf=1e6, eps=1e-5):
    """AttentionPairBias.forward (attentionv2.py:62-111) with k_in = s: q = s W_q^T + b_q, k = s W_k^T, v = s W_v^T, g = sigmoid(s W_g^T),
    bias = proj_z(z), attn = softmax_j(q.k / sqrt(D) + bias + (1 - mask[b, j]) * -inf), out = (g * (attn v)) W_o^T.
    s [B,N,c_s] (already normalised by the caller), z [B,N,N,c_z], mask [B,N] token mask."""
    ss = s.to(dtype)
    B, N, CS = ss.shape
    H = int(P["H"])
    D = CS // H
    q = (torch.matmul(ss, P["w_q"].to(dtype).t()) + P["b_q"].to(dtype)).view(B, N, H, D)
    k = torch.matmul(ss, P["w_k"].to(dtype).t()).view(B, N, H, D)
    v = torch.matmul(ss, P["w_v"].to(dtype).t()).view(B, N, H, D)
    bias = pair_bias(z, P["ln_z_w"], P["ln_z_b"], P["w_z"], eps=eps, dtype=dtype)
    g = torch.sigmoid(torch.matmul(ss, P["w_g"].to(dtype).t()))
    attn = torch.einsum("bihd,bjhd->bhij", q, k) / math.sqrt(D) + bias
    attn = attn + (1 - mask.to(dtype)[:, None, None, :]) * -inf
    attn = torch.softmax(attn, dim=-1)
    o = torch.einsum("bhij,bjhd->bihd", attn, v).reshape(B, N, CS)
    return torch.matmul(g * o, P["w_o"].to(dtype).t())


def single_track(s, z, mask, P, *, dtype=torch.float64, eps=1e-5):
    """The sequence stack of PairformerLayer.forward (pairformer.py:104-111, autocast off, post norm identity): s_n = LN_s(s);
    s += attention(s_n, z, mask, k_in = s_n); s += transition_s(s).  ``P`` = make_single_params(...)["apb"|"trs"] merged."""
    ss = s.to(dtype)
    a = P["apb"]
    sn = layer_norm(ss, a["ln_s_w"], a["ln_s_b"], eps)
    ss = ss + attention_pair_bias(sn, z, mask, a, dtype=dtype, eps=eps)
    t = P["trs"]
    return ss + transition(ss, t["w_a"], t["w_b"], t["w_o"], t["ln_w"], t["ln_b"], eps=eps, dtype=dtype)


def pairformer_layer(s, z, mask, pair_mask, params, *, dtype=torch.float64):
    """One PairformerLayer (pairformer.py:75-111, eval): the pair stack updates z, then the single track reads the updated z.
    Returns (s, z)."""
    z = pair_block(z, pair_mask, params, dtype=dtype)
    return single_track(s, z, mask, params["single"], dtype=dtype), z


def make_single_params(c_s=384, c_z=128, heads=16, factor=4, seed=0):
    """Single-track weights of one layer (N(0, 1/fan_in), LayerNorm 1 / 0, proj_q bias 0) in module order
    (pre_norm_s, proj_q, proj_k, proj_v, proj_g, proj_z, proj_o, transition_s).  fp32 CPU tensors."""
    g = torch.Generator("cpu").manual_seed(seed)

    def lin(o, i):
        return torch.randn(o, i, generator=g, dtype=torch.float32) / math.sqrt(i)
    apb = {"H": heads, "ln_s_w": torch.ones(c_s), "ln_s_b": torch.zeros(c_s), "w_q": lin(c_s, c_s), "b_q": torch.zeros(c_s),
           "w_k": lin(c_s, c_s), "w_v": lin(c_s, c_s), "w_g": lin(c_s, c_s), "ln_z_w": torch.ones(c_z), "ln_z_b": torch.zeros(c_z),
           "w_z": lin(heads, c_z), "w_o": lin(c_s, c_s)}
    hid = factor * c_s
    trs = {"ln_w": torch.ones(c_s), "ln_b": torch.zeros(c_s), "w_a": lin(hid, c_s), "w_b": lin(hid, c_s), "w_o": lin(c_s, hid)}
    return {"apb": apb, "trs": trs}


def single_flops(n, c_s=384, c_z=128, heads=16, factor=4):
    """Algorithmic FLOPs of one layer's single track: projections q|k|v|g|o 10 N c_s^2, attention 4 N^2 c_s, pair-bias producer
    2 N^2 c_z H, transition 6 factor N c_s^2."""
    return 10 * n * c_s * c_s + 4 * n * n * c_s + 2 * n * n * c_z * heads + 6 * factor * n * c_s * c_s

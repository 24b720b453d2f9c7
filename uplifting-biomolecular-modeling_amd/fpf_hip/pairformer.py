"""The Pairformer layer on a resident z: the five in-place pair sites in the reference order, then the single track.

Follows boltz2/stock/src/boltz/model/layers/pairformer.py:75-102 (trimul outgoing, trimul incoming, tri-att starting node,
tri-att ending node, transition_z; each ``z = z + f(z)``; dropout is the identity in eval) and the PAIRFUSE composition of
boltz2/opt/forward/pairfuse/bz_pairfuse.py:747-774 (one resident z updated in place by every site; the ending node reads z^T
by address).  Every site is one HIP entry point of libfpf_hip (trimul: 3 launches, tri-att: 3, transition: 1).

Parameter dicts (CPU or device tensors) per layer:
    tmo / tmi   the ten TriMul tensors (ln_in_w ln_in_b w_ag w_ap w_bg w_bp ln_out_w ln_out_b w_o w_og)
    tas / tae   ln_w ln_b w_q w_k w_v w_g [H*D, C] w_b [H, C] w_o [C, H*D] plus ints H, D
    tr          ln_w ln_b w_a w_b [n*C, C] w_o [C, n*C]
Single track (pairformer.py:104-111; ``random_single_params``): apb = pre_norm_s, proj_q (+ bias) / k / v / g [c_s, c_s], proj_z
(LayerNorm(c_z) + w_z [H, c_z]), proj_o; trs = transition_s.  It runs in fp32 like the stock sequence stack (autocast off): the
LayerNorm and transition kernels in their fp32 forms, the attention core ``fpf_apb_fwd`` (bias from the bf16 z by the producer
``fpf_apb_bias_fwd``), and the q|k|v|g / output projections as plain GEMMs through torch.
"""
import math

import torch

from .attn import apb_core as APB
from .attn import pair_fused as PF
from .kernels import ln as LN
from .kernels import transition as TR
from .kernels import trimul as TM

SITES = ("tmo", "tmi", "tas", "tae", "tr")


class PairBlock(object):
    """One layer's packed device weights (bf16 for word fast / big, fp32 for exact) and its TriMul caches."""

    def __init__(self, params, device, dtype):
        self.dtype = dtype
        dev = torch.device(device)

        def t(x, keep_f32=False):
            return x.detach().to(device=dev, dtype=torch.float32 if keep_f32 else dtype).contiguous()
        self.tmo = {k: t(v, k.startswith("ln_")) for k, v in params["tmo"].items()}
        self.tmi = {k: t(v, k.startswith("ln_")) for k, v in params["tmi"].items()}
        self.cache_o, self.cache_i = {}, {}
        self.ta = {}
        for site in ("tas", "tae"):
            p = params[site]
            self.ta[site] = PF.pack_triattn_weights(w_o=t(p["w_o"]), n_heads=int(p["H"]), head_dim=int(p["D"]), ln_w=t(p["ln_w"], True),
                                                    ln_b=t(p["ln_b"], True), w_q=t(p["w_q"]), w_k=t(p["w_k"]), w_v=t(p["w_v"]),
                                                    w_g=t(p["w_g"]), w_b=t(p["w_b"]))
        p = params["tr"]
        self.tr = TR.pack(w_o=t(p["w_o"]), w_a=t(p["w_a"]), w_b=t(p["w_b"]), ln_w=t(p["ln_w"], True), ln_b=t(p["ln_b"], True))


def pair_block(z, mask, blk, *, word="fast", rows=256, pair_bias=None):
    """z [B,N,N,C] (or [N,N,C]) updated in place by the five sites; returns z.  mask [B,N,N] / [N,N] (0/1) or None.
    ``pair_bias`` (the transition face's dict: w_z, out, ln_w, ln_b, eps): the single track's pair bias of the updated z, written
    to ``out`` by the transition kernel (word fast) or by the producer pass after the chunked transition (word big).

    ``word="big"`` is the memory-lean line of common/opt_core/opt_core/mem/chunk.py (the `big` levers), every site on blocks of
    ``rows`` rows, each bitwise equal to its whole-tensor form: the triangle multiplications in the rows mode (operand planes
    whole, the product plane for one row block: chunk.py:526), the triangle-attention blocks row-chunked after a bias pass over
    every pixel (chunk.py:424) and the transition in row blocks (chunk.py:370; its 4c hidden never leaves the chip either way)."""
    if word == "big":
        TM.triangle_multiplication_chunked(z, mask, direction="outgoing", weights=blk.tmo, chunk=rows, word=word, residual=True,
                                           cache=blk.cache_o, out=z)
        TM.triangle_multiplication_chunked(z, mask, direction="incoming", weights=blk.tmi, chunk=rows, word=word, residual=True,
                                           cache=blk.cache_i, out=z)
        PF.tri_attn_block_chunked(z, blk.ta["tas"], mask, ending=False, residual=True, chunk=rows, word=word)
        PF.tri_attn_block_chunked(z, blk.ta["tae"], mask, ending=True, residual=True, chunk=rows, word=word)
        TR.pair_transition_chunked(z, blk.tr, chunk=rows, word=word, residual=True, out=z)
        if pair_bias is not None:
            APB.pair_bias_producer(z, pair_bias["w_z"], pair_bias.get("ln_w"), pair_bias.get("ln_b"), eps=pair_bias.get("eps", 1e-5),
                                   out=pair_bias["out"])
        return z
    TM.triangle_multiplication(z, mask, direction="outgoing", weights=blk.tmo, word=word, residual=True, cache=blk.cache_o, out=z)
    TM.triangle_multiplication(z, mask, direction="incoming", weights=blk.tmi, word=word, residual=True, cache=blk.cache_i, out=z)
    PF.tri_attn_block(z, blk.ta["tas"], mask, ending=False, residual=True, word=word)
    PF.tri_attn_block(z, blk.ta["tae"], mask, ending=True, residual=True, word=word)
    TR.transition(z, blk.tr, word=word, residual=True, out=z, pair_bias=pair_bias)
    return z


def pair_stack(z, mask, blocks, *, word="fast", rows=256):
    """The pair part of a Pairformer trunk: ``pair_block`` over every layer of ``blocks`` (a list of PairBlock)."""
    for blk in blocks:
        pair_block(z, mask, blk, word=word, rows=rows)
    return z


class SingleBlock(object):
    """One layer's single-track weights on the device, fp32 (the stock sequence stack runs with autocast off): pre_norm_s, the
    AttentionPairBias module (q|k|v|g packed, proj_o, proj_z = LayerNorm + Linear(c_z -> H) with w_z in bf16 for the producer) and
    transition_s."""

    def __init__(self, params, device):
        dev = torch.device(device)
        a = params["apb"]
        self.ln_s_w = a["ln_s_w"].detach().to(device=dev, dtype=torch.float32).contiguous()
        self.ln_s_b = a["ln_s_b"].detach().to(device=dev, dtype=torch.float32).contiguous()
        self.apb = APB.ApbWeights(a, dev)
        t = params["trs"]
        f = lambda x: x.detach().to(device=dev, dtype=torch.float32).contiguous()      # noqa: E731
        self.tr = TR.pack(w_o=f(t["w_o"]), w_a=f(t["w_a"]), w_b=f(t["w_b"]), ln_w=f(t["ln_w"]), ln_b=f(t["ln_b"]))
        self.hidden = int(t["w_a"].shape[0])
        self.w_ab_t = torch.cat([f(t["w_a"]), f(t["w_b"])], 0).t().contiguous()       # [c_s, 2 hidden]: fc1 | fc2
        self.w_o_t = f(t["w_o"]).t().contiguous()                                       # [hidden, c_s]


def single_block(s, z, mask, sb, bias=None):
    """The sequence stack of one Pairformer layer (boltz2/stock/src/boltz/model/layers/pairformer.py:104-111, autocast off, post
    norm = identity): s_n = LN_s(s); s = s + AttentionPairBias(s_n, z, mask, k_in = s_n); s = s + transition_s(s).  s [B, N, c_s]
    fp32, z the bf16 pair tensor (already updated by this layer's pair stack), mask [B, N] token mask (or None), ``bias`` the pair
    bias of z when already produced (``pair_block(..., pair_bias=...)``).  Returns a new s."""
    c_s = s.shape[-1]
    s_n, _ = LN.layer_norm(s, c_s, sb.ln_s_w, sb.ln_s_b, 1e-5, word="exact")
    s = s + APB.attention_pair_bias_module(s_n, z, mask, sb.apb, bias=bias)
    # transition_s on N rows (transition.py:47-78): the LayerNorm kernel, then fc1 | fc2 in one library GEMM, silu * gate, fc3
    # and the residual add (plain GEMMs: N token rows are far too few for the fused transition kernels, built for N^2 pair rows)
    x_n, _ = LN.layer_norm(s, c_s, sb.tr.ln_w, sb.tr.ln_b, sb.tr.eps, word="exact")
    ab = torch.matmul(x_n, sb.w_ab_t)
    h = torch.nn.functional.silu(ab[..., :sb.hidden]) * ab[..., sb.hidden:]
    return s + torch.matmul(h, sb.w_o_t)


def pairformer_layer(s, z, mask, pair_mask, blk, sb, *, word="fast", rows=256):
    """One Pairformer layer (pairformer.py:64-113): the pair stack updates z in place, then the single track reads it.  The
    single track's pair bias is projected from z by the pair stack's last site (the transition) as it writes z, not by another
    pass over z.  Returns (s, z)."""
    z4 = z if z.dim() == 4 else z.unsqueeze(0)
    B, N = int(z4.shape[0]), int(z4.shape[1])
    bias = torch.empty((B, sb.apb.H, N, N), dtype=torch.float32, device=z.device)
    pb = dict(w_z=sb.apb.w_z, ln_w=sb.apb.ln_z_w, ln_b=sb.apb.ln_z_b, eps=1e-5, out=bias)
    pair_block(z, pair_mask, blk, word=word, rows=rows, pair_bias=pb)
    return single_block(s, z, mask, sb, bias=bias), z


def pairformer_trunk(s, z, mask, pair_mask, layers, *, word="fast", rows=256):
    """A Pairformer trunk (pairformer.py:116-200, eval): ``pairformer_layer`` over every (PairBlock, SingleBlock) of ``layers``."""
    for blk, sb in layers:
        s, z = pairformer_layer(s, z, mask, pair_mask, blk, sb, word=word, rows=rows)
    return s, z


def random_params(c_z=128, heads=4, head_dim=32, factor=4, seed=0):
    """Random-init weights of one layer (N(0, 1/fan_in) from torch.Generator('cpu').manual_seed(seed), LayerNorm 1 / 0), the
    BASELINE init: fp32 CPU tensors in the dict layout above."""
    g = torch.Generator("cpu").manual_seed(seed)
    C, H, D = c_z, heads, head_dim
    HD = H * D

    def lin(o, i):
        return torch.randn(o, i, generator=g, dtype=torch.float32) / math.sqrt(i)

    def tm():
        p_in, g_in, p_out, g_out = lin(2 * C, C), lin(2 * C, C), lin(C, C), lin(C, C)
        return {"ln_in_w": torch.ones(C), "ln_in_b": torch.zeros(C), "w_ap": p_in[:C], "w_bp": p_in[C:], "w_ag": g_in[:C],
                "w_bg": g_in[C:], "ln_out_w": torch.ones(C), "ln_out_b": torch.zeros(C), "w_o": p_out, "w_og": g_out}

    def ta():
        w_b = lin(H, C)
        w_q, w_k, w_v, w_o, w_g = lin(HD, C), lin(HD, C), lin(HD, C), lin(C, HD), lin(HD, C)
        return {"ln_w": torch.ones(C), "ln_b": torch.zeros(C), "w_q": w_q, "w_k": w_k, "w_v": w_v, "w_g": w_g, "w_b": w_b, "w_o": w_o,
                "H": H, "D": D}
    params = {"tmo": tm(), "tmi": tm(), "tas": ta(), "tae": ta()}
    hid = factor * C
    params["tr"] = {"ln_w": torch.ones(C), "ln_b": torch.zeros(C), "w_a": lin(hid, C), "w_b": lin(hid, C), "w_o": lin(C, hid)}
    return params


def random_single_params(c_s=384, c_z=128, heads=16, factor=4, seed=0):
    """Random-init single-track weights of one layer (N(0, 1/fan_in) from torch.Generator('cpu').manual_seed(seed),
    LayerNorm 1 / 0, proj_q bias 0), drawn in module order (proj_q, proj_k, proj_v, proj_g, proj_z, proj_o, transition_s fc1, fc2,
    fc3): {"apb": {...}, "trs": {...}} fp32 CPU tensors."""
    g = torch.Generator("cpu").manual_seed(seed)

    def lin(o, i):
        return torch.randn(o, i, generator=g, dtype=torch.float32) / math.sqrt(i)
    apb = {"H": heads, "ln_s_w": torch.ones(c_s), "ln_s_b": torch.zeros(c_s), "w_q": lin(c_s, c_s), "b_q": torch.zeros(c_s),
           "w_k": lin(c_s, c_s), "w_v": lin(c_s, c_s), "w_g": lin(c_s, c_s), "ln_z_w": torch.ones(c_z), "ln_z_b": torch.zeros(c_z),
           "w_z": lin(heads, c_z), "w_o": lin(c_s, c_s)}
    hid = factor * c_s
    trs = {"ln_w": torch.ones(c_s), "ln_b": torch.zeros(c_s), "w_a": lin(hid, c_s), "w_b": lin(hid, c_s), "w_o": lin(c_s, hid)}
    return {"apb": apb, "trs": trs}

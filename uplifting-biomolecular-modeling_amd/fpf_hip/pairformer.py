"""The Pairformer pair stack on a resident z: one layer = the five in-place pair sites, in the reference order.

Follows boltz2/stock/src/boltz/model/layers/pairformer.py:75-102 (trimul outgoing, trimul incoming, tri-att starting node,
tri-att ending node, transition_z; each ``z = z + f(z)``; dropout is the identity in eval) and the PAIRFUSE composition of
boltz2/opt/forward/pairfuse/bz_pairfuse.py:747-774 (one resident z updated in place by every site; the ending node reads z^T
by address).  Every site is one HIP entry point of libfpf_hip (trimul: 3 launches, tri-att: 3, transition: 1).

Parameter dicts (CPU or device tensors) per layer:
    tmo / tmi   the ten TriMul tensors (ln_in_w ln_in_b w_ag w_ap w_bg w_bp ln_out_w ln_out_b w_o w_og)
    tas / tae   ln_w ln_b w_q w_k w_v w_g [H*D, C] w_b [H, C] w_o [C, H*D] plus ints H, D
    tr          ln_w ln_b w_a w_b [n*C, C] w_o [C, n*C]
"""
import math

import torch

from .attn import pair_fused as PF
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


def pair_block(z, mask, blk, *, word="fast", rows=256):
    """z [B,N,N,C] (or [N,N,C]) updated in place by the five sites; returns z.  mask [B,N,N] / [N,N] (0/1) or None.

    ``word="big"`` is the memory-lean line of common/opt_core/opt_core/mem/chunk.py (the `big` levers): the triangle-attention
    blocks run row-chunked (``rows`` attention rows per launch; a bias pass over every pixel first), bitwise equal to the
    whole-tensor blocks.  The transition needs no chunking here (its 4c hidden never leaves the chip, so there is no per-row
    transient to bound) and triangle multiplication keeps its whole-plane contraction (3 c_h N^2 bf16 of workspace: 3.2 GB at
    N = 2048, far inside one MI355X's 288 GB)."""
    TM.triangle_multiplication(z, mask, direction="outgoing", weights=blk.tmo, word=word, residual=True, cache=blk.cache_o, out=z)
    TM.triangle_multiplication(z, mask, direction="incoming", weights=blk.tmi, word=word, residual=True, cache=blk.cache_i, out=z)
    if word == "big":
        PF.tri_attn_block_chunked(z, blk.ta["tas"], mask, ending=False, residual=True, chunk=rows, word=word)
        PF.tri_attn_block_chunked(z, blk.ta["tae"], mask, ending=True, residual=True, chunk=rows, word=word)
    else:
        PF.tri_attn_block(z, blk.ta["tas"], mask, ending=False, residual=True, word=word)
        PF.tri_attn_block(z, blk.ta["tae"], mask, ending=True, residual=True, word=word)
    TR.transition(z, blk.tr, word=word, residual=True, out=z)
    return z


def pair_stack(z, mask, blocks, *, word="fast", rows=256):
    """The pair part of a Pairformer trunk: ``pair_block`` over every layer of ``blocks`` (a list of PairBlock)."""
    for blk in blocks:
        pair_block(z, mask, blk, word=word, rows=rows)
    return z


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

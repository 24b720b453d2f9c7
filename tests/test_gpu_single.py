"""GPU parity of the single track: the attention-with-pair-bias core (``fpf_apb_fwd``) against the oracle's op statement, the
pair-bias producer (``fpf_apb_bias_fwd``) against the oracle's proj_z, and the Pairformer single track / full layer against the
stock statements (the single track runs fp32 like the stock sequence stack; the pair track bf16)."""
import math

import pytest
import torch

from _util import assert_bf16_close, assert_f32_close, assert_same_class, max_abs, rel_l2
from oracle import stock as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _apb_inputs(seed, S_, N, NK, H, D, per_sample, dtype):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(S_, n_, H, D, generator=g) for n_ in (N, NK, NK))
    bias = torch.randn(S_ if per_sample else 1, H, N, NK, generator=g)
    gate = torch.randn(S_, N, H, D, generator=g)
    return [t.to(dtype) for t in (q, k, v)] + [bias, gate.to(dtype)]


@pytest.mark.parametrize("D", [16, 24, 32, 48, 64])
@pytest.mark.parametrize("layout", ["rows", "shnd"])
@pytest.mark.parametrize("NK", [130, 128])
def test_apb_core_fp32(D, layout, NK):
    """fp32 against the fp64 statement; NK = 128 (16-byte aligned rows, a multiple of 4 keys) takes the kernel's 16-byte tile
    loads, NK = 130 the 4-byte ones."""
    from fpf_hip.attn import apb_core as APB
    S_, N, H = 2, 77, 3
    q, k, v, bias, gate = _apb_inputs(D, S_, N, NK, H, D, False, torch.float32)
    mask = (torch.arange(NK) % 5 != 3).to(torch.uint8).reshape(1, NK)
    ref = S.pair_bias_attention_op(q, k, v, bias, mask, gate, dtype=torch.float64).float()
    print("[apb] fp32 D=%d layout=%s NK=%d" % (D, layout, NK), flush=True)
    if layout == "rows":
        qd, kd, vd, gd = (t.reshape(-1, H * D).to(DEV) for t in (q, k, v, gate))
        out = APB.pair_bias_attention(qd, kd, vd, bias.to(DEV), mask.to(DEV), gate=gd, num_samples=S_, num_heads=H, layout="rows")
        out = out.reshape(S_, N, H, D)
    else:
        qd, kd, vd = (t.permute(0, 2, 1, 3).to(DEV) for t in (q, k, v))          # [S, H, N, D] views of [S, N, H, D] storage
        out = APB.pair_bias_attention(qd, kd, vd, bias.to(DEV), mask.to(DEV), gate=gate.to(DEV), layout="shnd").reshape(S_, N, H, D)
    torch.cuda.synchronize()
    assert_f32_close(out, ref, "apb fp32 D%d %s NK%d" % (D, layout, NK))


def test_apb_core_bf16_per_sample_bias_and_dead_sample():
    """bf16 storage, fp32 arithmetic: against the statement on the same bf16 values; sample 1 has every key masked (uniform mean)."""
    from fpf_hip.attn import apb_core as APB
    S_, N, NK, H, D = 3, 64, 100, 4, 24
    q, k, v, bias, gate = _apb_inputs(11, S_, N, NK, H, D, True, torch.bfloat16)
    bias = bias.to(torch.bfloat16)
    mask = torch.ones(S_, NK)
    mask[0, 90:] = 0
    mask[1] = 0
    mask[2, ::3] = 0
    ref = S.pair_bias_attention_op(q, k, v, bias, mask, gate, dtype=torch.float64)
    out = APB.pair_bias_attention(*(t.permute(0, 2, 1, 3).to(DEV) for t in (q, k, v)), bias.to(DEV), mask.to(DEV), gate=gate.to(DEV),
                                  layout="shnd").reshape(S_, N, H, D)
    torch.cuda.synchronize()
    # the output is rounded to bf16 once: half an ulp relative at most
    assert rel_l2(out, ref) <= 2.0 ** -9, rel_l2(out, ref)
    dead = out[1].float().cpu()
    uni = v[1].double().mean(dim=0)                                             # [H, D]
    assert max_abs(dead, (uni * torch.sigmoid(gate[1].double())).float()) <= 1e-2


def test_apb_core_one_key_is_v_and_shared_bias_equals_copies():
    from fpf_hip.attn import apb_core as APB
    S_, N, NK, H, D = 2, 40, 1, 2, 32
    q, k, v, bias, _ = _apb_inputs(12, S_, N, NK, H, D, False, torch.float32)
    out = APB.pair_bias_attention(*(t.permute(0, 2, 1, 3).to(DEV) for t in (q, k, v)), bias.to(DEV), layout="shnd").reshape(S_, N, H, D)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), v.expand(S_, N, H, D))
    q, k, v, bias, gate = _apb_inputs(13, 3, 50, 60, 2, 16, False, torch.float32)
    args = [t.permute(0, 2, 1, 3).to(DEV) for t in (q, k, v)]
    a = APB.pair_bias_attention(*args, bias.to(DEV), gate=gate.to(DEV), layout="shnd")
    b = APB.pair_bias_attention(*args, bias.expand(3, -1, -1, -1).contiguous().to(DEV), gate=gate.to(DEV), layout="shnd")
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_apb_refusals_by_name():
    from fpf_hip.attn import apb_core as APB
    q = torch.randn(1, 2, 8, 20, device=DEV)
    with pytest.raises(APB.Unsupported) as e:
        APB.pair_bias_attention(q, q, q, torch.zeros(2, 8, 8, device=DEV), layout="shnd")
    assert e.value.event == "head_dim:20"
    q = torch.randn(1, 2, 8, 24, device=DEV)
    with pytest.raises(APB.Unsupported) as e:
        APB.pair_bias_attention(q, q, q, torch.zeros(2, 8, 8, device=DEV), layout="shnd", inf=float("inf"))
    assert e.value.event == "nonfinite:inf_or_scale"
    assert APB.census()["refused"].get("head_dim:20", 0) >= 1


@pytest.mark.parametrize("out_dtype,pad", [(torch.float32, 0), (torch.bfloat16, 8)])
def test_pair_bias_producer(out_dtype, pad):
    from fpf_hip.attn import apb_core as APB
    g = torch.Generator().manual_seed(21)
    N, H = 70, 16
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16)
    w, b = 1 + 0.1 * torch.randn(128, generator=g), 0.1 * torch.randn(128, generator=g)
    wz = (torch.randn(H, 128, generator=g) / math.sqrt(128)).to(torch.bfloat16).float()
    ref = S.pair_bias(z.float(), w, b, wz, dtype=torch.float32)
    store = torch.full((1, H, N, N + pad), float("nan"), dtype=out_dtype, device=DEV)
    out = APB.pair_bias_producer(z.to(DEV), wz, w, b, out=store[..., :N])
    torch.cuda.synchronize()
    assert_bf16_close(out.float(), ref, "pair-bias producer %s pad %d" % (out_dtype, pad))
    if pad:
        assert torch.isnan(store[..., N:].float()).all()                            # the row padding is never written


@pytest.mark.parametrize("B,N,H,out_dtype,pad,masked", [(1, 96, 16, torch.float32, 0, False), (2, 130, 16, torch.bfloat16, 8, True),
                                                       (1, 768, 16, torch.float32, 0, True), (1, 37, 5, torch.float32, 3, False)])
def test_transition_pair_bias_equals_the_producer_on_the_written_z(B, N, H, out_dtype, pad, masked):
    """The pair bias projected by the transition kernel from the rows it writes (the single track's proj_z folded into the pair
    stack's last site) equals the producer's pass over the written z bitwise, and the written z equals the transition's without
    the bias: in place with the residual, a row mask, fp32 and bf16 bias with a padded row pitch, H below a 32-row block."""
    from fpf_hip import pairformer as PFM
    from fpf_hip.attn import apb_core as APB
    from fpf_hip.kernels import transition as TR
    g = torch.Generator().manual_seed(N + H)
    blk = PFM.PairBlock(PFM.random_params(seed=N), DEV, torch.bfloat16)
    z = torch.randn(B, N, N, 128, generator=g).to(torch.bfloat16).to(DEV)
    m = (torch.rand(B, N, N, generator=g) > 0.3).float().to(DEV) if masked else None
    wz = (torch.randn(H, 128, generator=g) / math.sqrt(128)).to(torch.bfloat16).to(DEV)
    lw, lb = (1 + 0.1 * torch.randn(128, generator=g)).to(DEV), (0.1 * torch.randn(128, generator=g)).to(DEV)
    print("[pair-bias] transition B=%d N=%d H=%d %s pad %d mask %s" % (B, N, H, out_dtype, pad, masked), flush=True)
    store = torch.full((B, H, N, N + pad), float("nan"), dtype=out_dtype, device=DEV)
    z1 = z.clone()
    TR.transition(z1, blk.tr, word="fast", residual=True, out=z1, mask=m,
                  pair_bias=dict(w_z=wz, ln_w=lw, ln_b=lb, eps=1e-5, out=store[..., :N]))
    z2 = z.clone()
    TR.transition(z2, blk.tr, word="fast", residual=True, out=z2, mask=m)
    ref = APB.pair_bias_producer(z2, wz, lw, lb, dtype=out_dtype)
    torch.cuda.synchronize()
    assert torch.equal(z1, z2), "the bias changed the written z"
    assert torch.equal(store[..., :N], ref), "max diff %.3e" % (store[..., :N].float() - ref.float()).abs().max().item()
    if pad:
        assert torch.isnan(store[..., N:].float()).all()                            # the row padding is never written


def test_transition_pair_bias_refusals():
    from fpf_hip import pairformer as PFM
    from fpf_hip.kernels import transition as TR
    blk = PFM.PairBlock(PFM.random_params(seed=1), DEV, torch.bfloat16)
    z = torch.randn(1, 16, 16, 128, device=DEV).to(torch.bfloat16)
    wz = torch.randn(4, 128, device=DEV).to(torch.bfloat16)
    good = torch.empty(1, 4, 16, 16, device=DEV)
    cases = [(dict(w_z=wz), "pair_bias:args"), (dict(w_z=torch.randn(40, 128, device=DEV), out=good), "pair_bias:w_z"),
             (dict(w_z=wz, out=torch.empty(1, 4, 16, 15, device=DEV)), "pair_bias:out"),
             (dict(w_z=wz, out=good.transpose(2, 3)), "pair_bias:out")]
    for pb, kind in cases:
        with pytest.raises(TR.Refusal) as e:
            TR.transition(z, blk.tr, word="fast", pair_bias=pb)
        assert e.value.kind == kind
    with pytest.raises(TR.Refusal) as e:
        TR.transition(z[0, :, :8].contiguous(), blk.tr, word="fast", pair_bias=dict(w_z=wz, out=good))
    assert e.value.kind == "pair_bias:not_pair"


def _layer(seed, N, c_s=384, heads=16):
    from fpf_hip import pairformer as PFM
    sp = PFM.random_single_params(c_s=c_s, heads=heads, seed=seed)
    for kk in ("w_q", "w_k", "w_v", "w_g", "w_o", "w_z"):                        # bf16-representable so both sides see the same values
        sp["apb"][kk] = sp["apb"][kk].to(torch.bfloat16).float()
    g = torch.Generator().manual_seed(seed + 1)
    s = torch.randn(1, N, c_s, generator=g)
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16)
    mask = torch.ones(1, N)
    mask[0, N - 5:] = 0
    return sp, s, z, mask


@pytest.mark.parametrize("N", [48, 512])
def test_single_block_against_the_stock_statement(N):
    """N = 512 is BASELINE config 3's single track (c_s = 384, 16 heads x 24)."""
    from fpf_hip import pairformer as PFM
    sp, s, z, mask = _layer(31, N)
    sb = PFM.SingleBlock(sp, DEV)
    print("[single] N=%d" % N, flush=True)
    out = PFM.single_block(s.to(DEV), z.to(DEV), mask.to(DEV), sb)
    torch.cuda.synchronize()
    ref = S.single_track(s, z.float(), mask, sp, dtype=torch.float32)
    # fp32 throughout except the pair bias, whose LayerNorm output is rounded to bf16 for the producer's MFMA (the stock
    # fp32 statement does not round): the fast-tier bars
    assert_bf16_close(out, ref, "single block N=%d" % N)


def test_pairformer_layer_against_the_stock_statement():
    from fpf_hip import pairformer as PFM
    N = 48
    sp, s, z, mask = _layer(41, N)
    params = PFM.random_params(seed=42)
    for site in ("tmo", "tmi", "tas", "tae", "tr"):
        for k_, v_ in params[site].items():
            if hasattr(v_, "dtype") and not k_.startswith("ln_"):
                params[site][k_] = v_.to(torch.bfloat16).float()
    pair_mask = mask[:, :, None] * mask[:, None, :]
    blk, sb = PFM.PairBlock(params, DEV, torch.bfloat16), PFM.SingleBlock(sp, DEV)
    zd = z.to(DEV)
    s_out, z_out = PFM.pairformer_layer(s.to(DEV), zd, mask.to(DEV), pair_mask.to(DEV), blk, sb, word="fast")
    torch.cuda.synchronize()
    ps = dict(params, single=sp)
    s_ref, z_ref = S.pairformer_layer(s, z.float(), mask, pair_mask, ps, dtype=torch.float32)
    # the yardstick: the stock layer with its pair stack under bf16 autocast (fp32 residual stream) and the fp32 single track
    z_ys = S.pair_block_autocast(z, pair_mask, params)
    s_ys = S.single_track(s, z_ys, mask, sp, dtype=torch.float32)
    assert_same_class(z_out.float(), z_ref, z_ys, "layer z N=%d" % N)
    assert_same_class(s_out, s_ref, s_ys, "layer s N=%d" % N)

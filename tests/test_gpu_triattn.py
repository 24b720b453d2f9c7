"""GPU parity of the triangle-attention core (op) and block (prologue -> core -> epilogue) against the CPU oracle."""
import json
import os

import numpy as np
import pytest
import torch

from _util import assert_bf16_close, assert_bf16_residual_close, assert_f32_close, max_abs, rel_l2
from conftest import GOLDEN
from oracle import stock as S
from oracle import vectors as V

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
CASES = json.load(open(os.path.join(GOLDEN, "triattn_cases.json")))["cases"]
BF16_CASES = [c for c in CASES if c["D"] == 32 and c["dtype"] == "bf16"]


def _to_dev(t):
    """Move a case's tensors to the GPU keeping strided views strided (the endstrided layout)."""
    out = {}
    for n in ("q", "k", "v"):
        x = t[n]
        if not x.is_contiguous():                       # [B,S,H,N,D] storage handed as a transposed view
            out[n] = x.transpose(1, 3).contiguous().to(DEV).transpose(1, 3)
        else:
            out[n] = x.to(DEV)
    out["bias"] = t["bias"].to(DEV)
    out["mask"] = None if t["mask"] is None else t["mask"].to(DEV)
    return out


@pytest.mark.parametrize("case", BF16_CASES, ids=[c["id"] for c in BF16_CASES])
def test_core_bf16_golden_cases(case):
    from fpf_hip.kernels import triattn as TA
    t = V.triattn_inputs(case)
    d = _to_dev(t)
    if case["layout"] == "endstrided":
        assert not d["q"].is_contiguous()
    out = TA.triangle_attention(d["q"], d["k"], d["v"], d["bias"], d["mask"], t["scale"], word="fast")
    torch.cuda.synchronize()
    ref32 = S.triangle_attention_op(t["q"], t["k"], t["v"], t["bias"], t["mask"], t["scale"], dtype=torch.float32)
    assert_bf16_close(out, ref32, case["id"])
    ref_row0 = torch.from_numpy(np.load(os.path.join(GOLDEN, "triattn_ref_%s.npy" % case["id"])))
    o0 = out[:, 0:1].float().cpu()
    print("[parity] %s row0 vs reference fp64: ours max_abs=%.3e | H100 recorded max_abs=%.3e (all rows)" % (
        case["id"], max_abs(o0, ref_row0), case["err_vs_fp64"]["max_abs"]))
    assert max_abs(o0, ref_row0) <= 2e-2


def test_core_head_dim_16_refused_by_bf16_row_and_served_by_fp32_row():
    from fpf_hip.kernels import triattn as TA
    case = [c for c in CASES if c["id"] == "a80_d16_s512_prefix"][0]
    t = V.triattn_inputs(case)
    with pytest.raises(TA.Refusal) as ei:
        TA.triangle_attention(t["q"].to(DEV), t["k"].to(DEV), t["v"].to(DEV), t["bias"].to(DEV), t["mask"].to(DEV), word="fast")
    assert ei.value.kind == "no_row:head_dim16" and ei.value.fallback == "hip_gfx950_f32"
    q, k, v = (t[n].float().to(DEV) for n in ("q", "k", "v"))
    out = TA.triangle_attention(q, k, v, t["bias"].to(DEV), t["mask"].to(DEV), t["scale"], word="exact")
    torch.cuda.synchronize()
    ref = S.triangle_attention_op(t["q"].double(), t["k"].double(), t["v"].double(), t["bias"], t["mask"], t["scale"], dtype=torch.float64)
    assert_f32_close(out, ref, "d16 fp32")


def _rand_op(B, N, H, Sq, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, N, H, Sq, D, generator=g).to(dtype) for _ in range(3))
    bias = (torch.randn(B, 1, H, Sq, Sq, generator=g) * 0.5)
    return q, k, v, bias


def test_core_bf16_dead_rows_are_uniform_mean():
    from fpf_hip.kernels import triattn as TA
    q, k, v, bias = _rand_op(1, 6, 4, 100, 32, 1, torch.bfloat16)
    mask = torch.ones(1, 6, 1, 1, 100, dtype=torch.bool)
    mask[0, 2] = False
    mask[0, 4, ..., 50:] = False
    out = TA.triangle_attention(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), mask.to(DEV), word="fast").cpu()
    ref = S.triangle_attention_op(q, k, v, bias, mask, dtype=torch.float32)
    assert_bf16_close(out, ref, "dead rows")
    mean = v[0, 2].float().mean(dim=-2, keepdim=True).expand(4, 100, 32)
    assert max_abs(out[0, 2], mean) <= 2 ** -8 * max(1.0, mean.abs().max().item())


def test_core_bf16_key_padding_is_bitwise_the_cropped_problem():
    """Valid queries of a key-padded call equal the cropped call bit for bit (masked keys contribute exact zeros)."""
    from fpf_hip.kernels import triattn as TA
    S_, L = 384, 346
    q, k, v, bias = _rand_op(1, 5, 4, S_, 32, 2, torch.bfloat16)
    mask = torch.zeros(1, 5, 1, 1, S_, dtype=torch.bool)
    mask[..., :L] = True
    full = TA.triangle_attention(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), mask.to(DEV), word="fast")
    crop = TA.triangle_attention(q[..., :L, :].contiguous().to(DEV), k[..., :L, :].contiguous().to(DEV), v[..., :L, :].contiguous().to(DEV),
                                 bias[..., :L, :L].contiguous().to(DEV), None, word="fast")
    torch.cuda.synchronize()
    assert torch.equal(full[..., :L, :], crop)


@pytest.mark.parametrize("S_,vt", [(800, False), (768, False), (456, True), (130, False)])
def test_op_face_staged_route_against_the_op_core_and_the_oracle(S_, vt):
    """The op face's staged route (bf16, head_dim 32, S a multiple of 64 or at least 128: q, V^T, bias and mask restaged for the
    block-layout core, S padded to a multiple of 64) against the same call without a workspace (the op core) and the fp32
    oracle, with a random keep mask, a dead row and a masked band; V given in [.., S, D] and transposed ([.., D, S] storage)."""
    from fpf_hip import _lib as L
    from fpf_hip.kernels import triattn as TA
    B, N, H, D = 1, 7, 4, 32
    q, k, v, bias = _rand_op(B, N, H, S_, D, 11, torch.bfloat16)
    g = torch.Generator().manual_seed(12)
    mask = torch.rand(B, N, 1, 1, S_, generator=g) > 0.2
    mask[0, 3] = False
    mask[0, 5, ..., S_ // 2:S_ // 2 + 40] = False
    assert L.lib().fpf_triattn_stage_bytes(B, N, H, S_, D, L.DT_BF16) > 0
    vd = v.to(DEV)
    if vt:
        vd = v.transpose(-1, -2).contiguous().to(DEV).transpose(-1, -2)          # V^T storage [B, N, H, D, S]
    print("[op staged] S=%d vt=%s" % (S_, vt), flush=True)
    staged = TA.triangle_attention(q.to(DEV), k.to(DEV), vd, bias.to(DEV), mask.to(DEV), word="fast")
    # the same call through the C ABI with no workspace: the op core
    out = torch.empty_like(staged)
    m8 = mask.reshape(B, N, S_).to(DEV).view(torch.uint8)
    qd, kd, bd = q.to(DEV), k.to(DEV), bias.to(DEV)
    a = L.TriattnArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, B=B, N=N, H=H, S=S_, D=D, q=L.ptr(qd), k=L.ptr(kd), v=L.ptr(vd),
                      bias=L.ptr(bd), bias_dtype=L.DT_F32, mask=L.ptr(m8), mask_dtype=L.DT_U8, out=L.ptr(out), scale=1.0 / D ** 0.5)
    a.q_stride[:] = list(qd.stride())
    a.k_stride[:] = list(kd.stride())
    vs = list(vd.stride())
    a.v_stride[:] = [vs[0], vs[1], vs[2], vs[4], vs[3]] if vt else vs
    a.v_layout = 1 if vt else 0
    a.out_stride[:] = list(out.stride())
    bs = list(bd.stride())
    a.bias_stride[:] = [bs[0], bs[2], bs[3], bs[4]]
    a.mask_stride[:] = list(m8.stride())
    L.call("fpf_triattn_fwd", a, L.stream_ptr(DEV))
    torch.cuda.synchronize()
    assert torch.isfinite(staged.float()).all()
    ref = S.triangle_attention_op(q, k, v, bias, mask, dtype=torch.float32)
    assert_bf16_close(staged, ref, "staged S=%d vt=%s" % (S_, vt))
    assert_bf16_close(out, ref, "op core S=%d vt=%s" % (S_, vt))
    mean = v[0, 3].float().mean(dim=-2, keepdim=True).expand(H, S_, D)
    assert max_abs(staged[0, 3].cpu(), mean) <= 2 ** -8 * max(1.0, mean.abs().max().item())


def test_core_bf16_run_to_run_bitwise():
    from fpf_hip.kernels import triattn as TA
    q, k, v, bias = (t.to(DEV) for t in _rand_op(1, 8, 4, 200, 32, 3, torch.bfloat16))
    a = TA.triangle_attention(q, k, v, bias, None, word="fast")
    b = TA.triangle_attention(q, k, v, bias, None, word="fast")
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("D", [32, 64])
def test_core_fp32_exact(D):
    from fpf_hip.kernels import triattn as TA
    q, k, v, bias = _rand_op(1, 4, 2, 150, D, 4, torch.float32)
    mask = torch.ones(1, 4, 1, 1, 150, dtype=torch.bool)
    mask[0, 1, ..., 120:] = False
    mask[0, 3] = False
    out = TA.triangle_attention(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), mask.to(DEV), word="exact")
    torch.cuda.synchronize()
    ref = S.triangle_attention_op(q, k, v, bias, mask, dtype=torch.float64)
    assert_f32_close(out, ref, "core fp32 D%d" % D)


# ------------------------------------------------------------------------------------------------------------------ block
def _block_weights(dtype, seed=0):
    P = S.make_block_params(c_z=128, heads=4, head_dim=32, seed=seed)["tas"]
    g = torch.Generator().manual_seed(seed + 100)
    P["ln_w"] = 1 + 0.1 * torch.randn(128, generator=g)
    P["ln_b"] = 0.1 * torch.randn(128, generator=g)
    for n in ("w_q", "w_k", "w_v", "w_g", "w_b", "w_o"):
        P[n] = P[n].to(dtype).float()                 # bf16-representable weights: the oracle and the kernel see the same values
    return P


def _pack(P, dtype):
    from fpf_hip.attn import pair_fused as PF
    return PF.pack_triattn_weights(w_o=P["w_o"].to(DEV), n_heads=4, head_dim=32, ln_w=P["ln_w"].to(DEV), ln_b=P["ln_b"].to(DEV),
                                   w_q=P["w_q"].to(DEV), w_k=P["w_k"].to(DEV), w_v=P["w_v"].to(DEV), w_g=P["w_g"].to(DEV), w_b=P["w_b"].to(DEV))


@pytest.mark.parametrize("ending", [False, True])
@pytest.mark.parametrize("N,pad", [(64, 0), (96, 10), (37, 3), (128, 10), (192, 70)])
def test_block_bf16(ending, N, pad):
    from fpf_hip.attn import pair_fused as PF
    P = _block_weights(torch.bfloat16)
    W = _pack(P, torch.bfloat16)
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(N)).to(torch.bfloat16)
    mask = torch.ones(1, N, N)
    if pad:
        mask[:, N - pad:, :] = 0
        mask[:, :, N - pad:] = 0
    u = PF.tri_attn_block(z.to(DEV), W, mask.to(DEV), ending=ending, residual=False)
    torch.cuda.synchronize()
    ref = S.tri_attn(z.float(), P, mask, ending=ending, dtype=torch.float32)
    assert_bf16_close(u, ref, "block ending=%s N%d pad%d" % (ending, N, pad))
    zz = z.to(DEV).clone()
    r = PF.tri_attn_block(zz, W, mask.to(DEV), ending=ending, residual=True)
    torch.cuda.synchronize()
    assert r.data_ptr() == zz.data_ptr()
    assert_bf16_residual_close(zz, z.float() + ref, "block residual ending=%s" % ending)


def _block_abi(z4, W, m, mdt, mframe, ending):
    """fpf_triattn_block_fwd called directly with a caller-chosen mask tensor, dtype and frame."""
    from fpf_hip import _lib as L
    from fpf_hip.attn import pair_fused as PF
    B, N = int(z4.shape[0]), int(z4.shape[1])
    wqkvg, wb, wo, bg, bo = PF._wpack(W, z4.dtype, z4.device)
    ws = torch.empty(L.lib().fpf_triattn_block_workspace_bytes(B, N, 0, W.C, W.H, W.D, L.DT_BF16), dtype=torch.uint8, device=z4.device)
    out = torch.empty_like(z4)
    a = L.TriattnBlockArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, B=B, N=N, C=W.C, H=W.H, D=W.D, z=L.ptr(z4), mask=L.ptr(m), mask_dtype=mdt,
                           ln_w=L.ptr(W.ln_w), ln_b=L.ptr(W.ln_b), eps=W.eps, w_qkvg=L.ptr(wqkvg), w_b=L.ptr(wb), w_o=L.ptr(wo),
                           ending=int(ending), residual=0, out=L.ptr(out), scale=0.0, workspace=L.ptr(ws), workspace_bytes=ws.numel(),
                           mask_frame=mframe, b_g=L.ptr(bg), b_o=L.ptr(bo))
    L.call("fpf_triattn_block_fwd", a, L.stream_ptr(z4.device))
    return out


@pytest.mark.parametrize("ending", [False, True])
@pytest.mark.parametrize("N", [100, 128])
def test_block_bf16_mask_frames_asymmetric_mask(ending, N):
    """An asymmetric pair mask (a transposed key mask would be caught, unlike the symmetric padding masks above) given in
    the z frame (mask_frame 0, u8 and fp32: the ending node reads key k of row i at mask[k, i]) is bitwise the attention-frame
    u8 mask the pair stack passes (mask_frame 1), and all match the oracle.  N = 128 takes the 64-key DMA core with the
    16-byte keep-table loads; N = 100 the generic core."""
    from fpf_hip import _lib as L
    from fpf_hip.attn import pair_fused as PF
    P = _block_weights(torch.bfloat16, seed=3)
    W = _pack(P, torch.bfloat16)
    g = torch.Generator().manual_seed(N + 7)
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16)
    mask = (torch.rand(1, N, N, generator=g) > 0.3).float()
    mask[:, :, N - 5:] = 0                               # whole key columns off on one side only
    print("[case] mask frames ending=%s N=%d" % (ending, N), flush=True)
    zd, md = z.to(DEV), mask.to(DEV)
    u = PF.tri_attn_block(zd, W, md, ending=ending, residual=False)
    u_z8 = _block_abi(zd, W, (md != 0).view(torch.uint8).contiguous(), L.DT_U8, 0, ending)
    u_zf = _block_abi(zd, W, md.contiguous(), L.DT_F32, 0, ending)
    torch.cuda.synchronize()
    assert torch.equal(u.view_as(u_z8), u_z8), "z-frame u8 mask differs from the attention-frame mask"
    assert torch.equal(u_z8, u_zf), "u8 and fp32 z-frame masks differ"
    ref = S.tri_attn(z.float(), P, mask, ending=ending, dtype=torch.float32)
    assert_bf16_close(u, ref, "block asymmetric mask ending=%s N%d" % (ending, N))
    with pytest.raises(L.LibError):
        _block_abi(zd, W, md.contiguous(), L.DT_F32, 2, ending)


@pytest.mark.parametrize("ending", [False, True])
def test_block_keep_table_builders_agree(ending):
    """The keep table's two builders -- 16-byte loads for a contiguous u8 mask (attention frame), one byte per lane for an
    fp32 or strided mask (z frame) -- give the same block output bit for bit at N = 1088 (keys past 1024: a second load
    round), with a dead row (no key kept: uniform attention) and a fully kept row next to a random pattern."""
    from fpf_hip import _lib as L
    P = _block_weights(torch.bfloat16, seed=5)
    W = _pack(P, torch.bfloat16)
    N = 1088
    g = torch.Generator().manual_seed(11)
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16)
    mask = (torch.rand(1, N, N, generator=g) > 0.25).float()
    mask[:, 7, :] = 0                                    # row 7: no key kept
    mask[:, 9, :] = 1                                    # row 9: every key kept
    mask[:, :, N - 70:] = 0                              # the last keys (the second load round) off
    print("[case] keep builders ending=%s N=%d" % (ending, N), flush=True)
    zd, md = z.to(DEV), mask.to(DEV)
    att = (md.transpose(1, 2) if ending else md) != 0
    u_a8 = _block_abi(zd, W, att.view(torch.uint8).contiguous(), L.DT_U8, 1, ending)
    u_zf = _block_abi(zd, W, md.contiguous(), L.DT_F32, 0, ending)
    torch.cuda.synchronize()
    assert torch.equal(u_a8, u_zf), "the u8 and fp32 keep-table builders differ"
    assert torch.isfinite(u_a8.float()).all()


@pytest.mark.parametrize("ending", [False, True])
def test_block_fp32_exact(ending):
    from fpf_hip.attn import pair_fused as PF
    P = _block_weights(torch.float32, seed=1)
    W = _pack(P, torch.float32)
    N = 40
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(9))
    mask = torch.ones(1, N, N)
    mask[:, :, N - 4:] = 0
    u = PF.tri_attn_block(z.to(DEV), W, mask.to(DEV), ending=ending, residual=False, word="exact")
    torch.cuda.synchronize()
    ref = S.tri_attn(z, P, mask, ending=ending, dtype=torch.float64)
    live = slice(0, N - 4) if ending else slice(0, N)
    assert_f32_close(u[:, :, live] if ending else u, ref[:, :, live] if ending else ref, "block fp32 ending=%s" % ending)


# ------------------------------------------------------------------------------------------------------------------ block stages
@pytest.mark.parametrize("ending", [False, True])
def test_stages_bf16_prologue_core_epilogue(ending):
    """prologue / core_attention / epilogue as separate faces: each stage against the oracle's stage, and the chain bitwise equal
    to the fused block (same kernels, same intermediate layout)."""
    from fpf_hip.attn import pair_fused as PF
    P = _block_weights(torch.bfloat16, seed=3)
    W = _pack(P, torch.bfloat16)
    N = 80
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(31)).to(torch.bfloat16)
    mask = torch.ones(1, N, N)
    mask[:, N - 6:, :] = 0
    mask[:, :, N - 6:] = 0
    zd, md = z.to(DEV), mask.to(DEV)
    print("[case] stages bf16 ending=%s N=%d" % (ending, N), flush=True)
    q, k, v, g, bias = PF.prologue(zd, W, ending=ending)
    torch.cuda.synchronize()
    assert v.stride(-1) != 1 and v.stride(-2) == 1          # V handed over transposed, served without a copy
    rq, rk, rv, rg, rb = S.triatt_prologue(z.float(), P, ending=ending, dtype=torch.float32)
    for name, got, ref in (("q", q, rq), ("k", k, rk), ("v", v, rv), ("g", g, rg), ("bias", bias, rb)):
        assert tuple(got.shape) == tuple(ref.shape), name
        if name == "bias":                                    # fp32 output
            assert_bf16_close(got, ref, "prologue %s ending=%s" % (name, ending))
        else:                                                 # bf16 outputs: half an output ulp on top of the bar
            assert_bf16_residual_close(got, ref, "prologue %s ending=%s" % (name, ending))
    o = PF.core_attention(q, k, v, bias, PF._key_mask(md, zd, ending), core="tier:fast")
    u = PF.epilogue(o, g, W, zd, ending=ending, residual=False)
    torch.cuda.synchronize()
    ref_o = S.triangle_attention_op(q.float().cpu(), k.float().cpu(), v.float().cpu(), bias.cpu(),
                                    PF._key_mask(mask, z, ending), dtype=torch.float32)
    assert_bf16_close(o, ref_o, "core on the prologue's tensors ending=%s" % ending)
    ref_u = S.triatt_epilogue(o.float().cpu(), g.float().cpu(), P, dtype=torch.float32)
    assert_bf16_residual_close(u, ref_u, "epilogue ending=%s" % ending)
    # the fused block recomputes the gate from z in fp32 (the staged chain reads the stored bf16 g): same statement, one
    # rounding fewer, so the two agree to bf16 tolerance rather than bitwise; both are held to the oracle
    blk = PF.tri_attn_block(zd, W, md, ending=ending, residual=False)
    torch.cuda.synchronize()
    ref_blk = S.tri_attn(z.float(), P, mask, ending=ending, dtype=torch.float32)
    assert_bf16_close(blk, ref_blk, "fused block ending=%s" % ending)
    assert_bf16_close(u.transpose(1, 2) if ending else u, blk.float(), "staged chain vs fused block ending=%s" % ending)
    zz = zd.clone()
    r = PF.epilogue(o, g, W, zz, ending=ending, residual=True)
    torch.cuda.synchronize()
    assert r.data_ptr() == zz.data_ptr()
    assert_bf16_residual_close(zz, z.float() + (u.transpose(1, 2) if ending else u).float().cpu(), "staged residual ending=%s" % ending)


def test_stages_fp32_exact():
    from fpf_hip.attn import pair_fused as PF
    P = _block_weights(torch.float32, seed=4)
    W = _pack(P, torch.float32)
    N = 24
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(41))
    print("[case] stages fp32 N=%d" % N, flush=True)
    for ending in (False, True):
        q, k, v, g, bias = PF.prologue(z.to(DEV), W, ending=ending, word="exact")
        torch.cuda.synchronize()
        for name, got, ref in zip(("q", "k", "v", "g", "bias"), (q, k, v, g, bias), S.triatt_prologue(z, P, ending=ending, dtype=torch.float64)):
            assert_f32_close(got, ref, "prologue fp32 %s ending=%s" % (name, ending))
        o = PF.core_attention(q, k, v, bias, None, core="tier:exact")
        u = PF.epilogue(o, g, W, ending=ending, residual=False, word="exact")
        torch.cuda.synchronize()
        ref = S.tri_attn(z, P, None, ending=ending, dtype=torch.float64)
        assert_f32_close(u.transpose(1, 2) if ending else u, ref, "staged fp32 ending=%s" % ending)


# ------------------------------------------------------------------------------------------------ block-layout core fallback
_VPERM = [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]      # stored position p of a 16-key block holds key _VPERM[p]


def _bias_blocks(bias):
    """[B, H, S, S] fp32 bias (query, key) -> the block-layout core's planes (csrc/triattn.h, bias_blk_off): 32 x 32 blocks
    (query block, key block) in row-major block order, each as pieces j (keys 8j .. 8j+7) x lanes n + 32g (query n, keys
    8j + 4g .. +3) x 4; returned with the shape and strides of a contiguous [B, H, S, S] tensor."""
    B, H, S, _ = bias.shape
    v = bias.reshape(B, H, S // 32, 32, S // 32, 4, 2, 4)                    # b, h, qt, n, kt, j, g, e
    return v.permute(0, 1, 2, 4, 5, 6, 3, 7).contiguous().view(B, H, S, S)


def _keep_table(mask, real=None):
    """The keep-bit table of the block-layout core (include/fpf_hip.h, FpfTriattnArgs.keep), built on the host from a [B, N, S]
    0/1 mask: per attention row, word 0 = flags (1 some key kept, 2 every key kept), word 1 + t = bits of keys 64 t .. 64 t + 63;
    a row with no kept key has the bit of every real key (the first `real`, default all) set."""
    B, N, S = mask.shape
    real = S if real is None else real
    m = (mask != 0).cpu().numpy().reshape(B, N, S // 64, 64).astype(np.uint64)
    words = (m << np.arange(64, dtype=np.uint64)).sum(axis=-1, dtype=np.uint64)
    alive = m.reshape(B, N, S).any(axis=-1)
    full = m.reshape(B, N, S).all(axis=-1)
    r = (np.arange(S) < real).astype(np.uint64).reshape(S // 64, 64)
    words[~alive] = (r << np.arange(64, dtype=np.uint64)).sum(axis=-1, dtype=np.uint64)
    flags = alive.astype(np.uint64) | (full.astype(np.uint64) << np.uint64(1))
    table = np.concatenate([flags[..., None], words], axis=-1)
    return torch.from_numpy(table.view(np.int64).copy()).to(DEV)


@pytest.mark.parametrize("N", [256, 768])
@pytest.mark.parametrize("masked,vrows", [(False, False), (True, False), (True, True)])
def test_block_layout_core_fallback_extreme_logits(N, masked, vrows):
    """The block's own core layout (v_layout 2, logits in log2 units) with query tiles whose logits need a reference max other
    than 0: bias +150 on queries 64..127 (a partial row sum far above 2^64) and -120 on queries 192..255 (every logit of a
    query's first sub-tile below -32), next to ordinary query tiles.  The fast kernel flags the work items of the extreme
    tiles and the fallback recomputes them; every sampled row is held to the bf16 bars against a max-subtracted fp32 softmax.
    N = 256 takes the 4-wave split, N = 768 the 8-wave one; `masked` adds a random keep pattern with dead rows (uniform mean);
    `vrows` hands V as key rows (v_layout 3) instead of V^T in the core's key order (v_layout 2)."""
    import ctypes
    from fpf_hip import _lib as L
    H, D = 4, 32
    g = torch.Generator().manual_seed(N + masked)
    q = (torch.randn(1, N, H, N, D, generator=g) / np.sqrt(D)).to(torch.bfloat16).to(DEV)
    k = torch.randn(1, N, H, N, D, generator=g).to(torch.bfloat16).to(DEV)
    vt = torch.randn(1, N, H, D, N, generator=g).to(torch.bfloat16).to(DEV)
    bias = torch.randn(1, H, N, N, generator=g) * 0.5
    bias[:, :, 64:128, :] += 150.0
    bias[:, :, 192:256, :] -= 120.0
    bias = bias.to(DEV)
    mask = keep = None
    if masked:
        mask = (torch.rand(1, N, N, generator=g) > 0.3).float()
        mask[:, 5:9, :] = 0                                                   # dead rows
        mask = mask.to(DEV)
        keep = _keep_table(mask)
    out = torch.full((1, N, H, N, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(max(1, L.lib().fpf_triattn_workspace_bytes(1, N, H, N, 2)), dtype=torch.uint8, device=DEV)
    bias_blk = _bias_blocks(bias)
    idx = torch.tensor([16 * (kk // 16) + _VPERM.index(kk % 16) for kk in range(N)], device=DEV)
    vin = vt[..., idx].transpose(-1, -2).contiguous() if vrows else vt           # key rows [1, N, H, key, D]
    a = L.TriattnArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, B=1, N=N, H=H, S=N, D=D, q=L.ptr(q), k=L.ptr(k), v=L.ptr(vin),
                      v_layout=3 if vrows else 2, bias=L.ptr(bias_blk), bias_dtype=L.DT_F32, mask=L.ptr(mask), mask_dtype=L.DT_F32,
                      out=L.ptr(out), scale=1.0, keep=None if keep is None else ctypes.c_void_p(keep.data_ptr()),
                      workspace=L.ptr(ws), workspace_bytes=ws.numel())
    a.q_stride[:] = q.stride()
    a.k_stride[:] = k.stride()
    a.v_stride[:] = vin.stride()
    a.out_stride[:] = out.stride()
    a.bias_stride[:] = bias_blk.stride()
    if masked:
        a.mask_stride[:] = mask.stride()
    print("[fallback] N=%d masked=%s vrows=%s" % (N, masked, vrows), flush=True)
    L.call("fpf_triattn_fwd", a, L.stream_ptr(DEV))
    torch.cuda.synchronize()
    rows = sorted(set([0, 1, 2, 5, 6, 7, 8, 9, N // 2, N // 2 + 1, N - 2, N - 1]))
    Vl = vt[0, rows].float()[..., idx].transpose(-1, -2)                   # [rows, H, key, D]
    s = torch.einsum("ihqd,ihkd->ihqk", q[0, rows].float(), k[0, rows].float()) + bias[0].unsqueeze(0)
    if masked:
        km = mask[0, rows] != 0                                              # [rows, key]
        dead = ~km.any(-1)
        s = torch.where(km[:, None, None, :] | dead[:, None, None, None], s, torch.full_like(s, -float("inf")))
        s = torch.where(dead[:, None, None, None], torch.zeros_like(s), s)
    p = torch.exp2(s - s.amax(-1, keepdim=True))
    ref = torch.einsum("ihqk,ihkd->ihqd", p / p.sum(-1, keepdim=True), Vl)
    got = out[0, rows].float()
    assert torch.isfinite(got).all(), "non-finite output"
    assert_bf16_close(got, ref, "block-layout core N=%d masked=%s vrows=%s, extreme query tiles" % (N, masked, vrows))


@pytest.mark.parametrize("S_,layout,N,B,bias_bf16", [(456, "contig", 7, 1, False), (800, "contig", 7, 1, False),
                                                     (768, "endstrided", 7, 1, False), (130, "endstrided", 7, 1, False),
                                                     (720, "contig", 512, 1, False), (300, "endstrided", 5, 2, False),
                                                     (200, "contig", 6, 1, True)])
def test_op_face_in_place_route_equals_the_block_core_on_restaged_operands(S_, layout, N, B, bias_bf16):
    """The op face's route onto the block-layout core reads q, k and v in place -- q times scale * log2(e) in registers, V's
    key rows through LDS transpose reads, the padding keys of the last tile re-reading the last real key row under the keep
    table's mask -- and restages only the bias.  Its output equals, bit for bit, the block-layout core with V^T in its key
    order (v_layout 2) given every operand restaged on the host:
    q2 = bf16(q * fp32(scale * log2(e))), k and V^T padded with zeros to Sp = S rounded up to 64 (V^T in the 16-block key
    order), the bias times log2(e) in register-order blocks, the keep table with the padding keys masked.  A random mask with a
    dead row; `endstrided`: q, k and v as transposed views of [B, S, H, N, D] storage (the ending node's layout).  N = 7 runs the
    4-wave split, N = 512 at S = 720 (padded to 768) the 8-wave one; B = 2 runs two batch entries; `bias_bf16` hands the
    bias as bf16 (restaged as its fp32 value times log2(e))."""
    import ctypes
    from fpf_hip import _lib as L
    from fpf_hip.kernels import triattn as TA
    H, D = 4, 32
    Sp = -(-S_ // 64) * 64
    q, k, v, bias = _rand_op(B, N, H, S_, D, 31 + S_, torch.bfloat16)
    if bias_bf16:
        bias = bias.to(torch.bfloat16)
    g = torch.Generator().manual_seed(32 + S_)
    mask = torch.rand(B, N, 1, 1, S_, generator=g) > 0.2
    mask[0, 3] = False
    mask[B - 1, 1, ..., S_ // 3:] = False
    if layout == "endstrided":
        qd, kd, vd = (t.transpose(1, 3).contiguous().to(DEV).transpose(1, 3) for t in (q, k, v))
    else:
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    print("[op in place] S=%d %s N=%d B=%d" % (S_, layout, N, B), flush=True)
    got = TA.triangle_attention(qd, kd, vd, bias.to(DEV), mask.to(DEV), word="fast")
    # every operand restaged on the host, for the core's own layout
    qmul = float(np.float32(np.float32(1.0 / np.sqrt(D)) * np.float32(1.4426950408889634)))
    q2 = torch.zeros(B, N, H, Sp, D, dtype=torch.bfloat16)
    q2[..., :S_, :] = (q.float() * qmul).to(torch.bfloat16)
    k2 = torch.zeros(B, N, H, Sp, D, dtype=torch.bfloat16)
    k2[..., :S_, :] = k
    vT = torch.zeros(B, N, H, D, Sp, dtype=torch.bfloat16)
    vT[..., :S_] = v.transpose(-1, -2)
    perm = torch.tensor([16 * (p // 16) + _VPERM[p % 16] for p in range(Sp)])
    v2 = vT[..., perm].contiguous()
    b2 = torch.zeros(B, H, Sp, Sp)
    b2[:, :, :S_, :S_] = bias[:, 0].float() * float(np.float32(1.4426950408889634))
    b2 = _bias_blocks(b2).to(DEV)
    m2 = torch.zeros(B, N, Sp)
    m2[..., :S_] = mask.reshape(B, N, S_).float()
    keep = _keep_table(m2, real=S_)
    q2, k2, v2 = q2.to(DEV), k2.to(DEV), v2.to(DEV)
    out = torch.full((B, N, H, Sp, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(max(1, L.lib().fpf_triattn_workspace_bytes(B, N, H, Sp, 2)), dtype=torch.uint8, device=DEV)
    a = L.TriattnArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, B=B, N=N, H=H, S=Sp, D=D, q=L.ptr(q2), k=L.ptr(k2), v=L.ptr(v2),
                      v_layout=2, bias=L.ptr(b2), bias_dtype=L.DT_F32, out=L.ptr(out), scale=1.0,
                      keep=ctypes.c_void_p(keep.data_ptr()), workspace=L.ptr(ws), workspace_bytes=ws.numel())
    a.q_stride[:] = q2.stride()
    a.k_stride[:] = k2.stride()
    a.v_stride[:] = v2.stride()
    a.out_stride[:] = out.stride()
    a.bias_stride[:] = b2.stride()
    L.call("fpf_triattn_fwd", a, L.stream_ptr(DEV))
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, out[..., :S_, :]), "in-place route differs from the restaged core: max |d| %g" % max_abs(
        got.float().cpu(), out[..., :S_, :].float().cpu())


def _xln_weights(seed):
    P = S.make_block_params(c_z=128, heads=4, head_dim=32, seed=seed)["tas"]
    g = torch.Generator().manual_seed(seed + 100)
    P["ln_w"] = 1 + 0.1 * torch.randn(128, generator=g)
    P["ln_b"] = 0.1 * torch.randn(128, generator=g)
    for n in ("w_q", "w_k", "w_v", "w_g", "w_b", "w_o"):
        P[n] = P[n].to(torch.bfloat16).float()
    return P


@pytest.mark.parametrize("ending", [False, True])
@pytest.mark.parametrize("N,residual", [(96, False), (300, True)])
def test_block_bf16_ln_stock_x_ln(ending, N, residual):
    """ln="stock" with x_ln (pair_fused.py:1019-1029, :1151-1160): the caller's own LayerNorm output in the attention frame is
    projected for q, k, v, the bias and the gate instead of the in-kernel LayerNorm of z, and the residual still updates z.  Here
    x_ln = bf16(LN(x) * 1.05 + 0.02), so a kernel that normalised z itself would be caught; against the statement with that x_ln,
    through the fused block and through the staged route (a callable core between the prologue and the epilogue)."""
    from fpf_hip.attn import pair_fused as PF
    P = _xln_weights(81)
    W = PF.pack_triattn_weights(w_o=P["w_o"].to(DEV, torch.bfloat16), n_heads=4, head_dim=32, ln_w=P["ln_w"].to(DEV), ln_b=P["ln_b"].to(DEV),
                                w_q=P["w_q"].to(DEV, torch.bfloat16), w_k=P["w_k"].to(DEV, torch.bfloat16),
                                w_v=P["w_v"].to(DEV, torch.bfloat16), w_g=P["w_g"].to(DEV, torch.bfloat16), w_b=P["w_b"].to(DEV, torch.bfloat16))
    g = torch.Generator().manual_seed(82)
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16)
    mask = torch.ones(1, N, N)
    mask[:, :, N - 9:] = 0
    x = z.transpose(1, 2) if ending else z
    xl = (S.layer_norm(x.float(), P["ln_w"], P["ln_b"], 1e-5) * 1.05 + 0.02).to(torch.bfloat16).contiguous()
    print("[x_ln] block N=%d ending=%s residual=%s" % (N, ending, residual), flush=True)
    zd, md, xd = z.to(DEV), mask.to(DEV), xl.to(DEV)
    u = PF.tri_attn_block(zd.clone(), W, md, ending=ending, residual=residual, ln="stock", x_ln=xd)
    fused = PF.tri_attn_block(zd.clone(), W, md, ending=ending, residual=residual)

    def torch_core(q, k, v, bias, m5, scale):
        o = S.triangle_attention_op(q.cpu(), k.cpu(), v.cpu(), bias.cpu(), None if m5 is None else m5.cpu(), scale, dtype=torch.float32)
        return o.to(q.device, q.dtype)
    staged = PF.tri_attn_block(zd.clone(), W, md, ending=ending, residual=residual, ln="stock", x_ln=xd, core=torch_core)
    torch.cuda.synchronize()
    ref = S.tri_attn(z.float(), P, mask, ending=ending, dtype=torch.float32, x_ln=xl.float())
    check = assert_bf16_residual_close if residual else assert_bf16_close
    want = z.float() + ref if residual else ref
    check(u, want, "x_ln block N=%d ending=%s" % (N, ending))
    check(staged, want, "x_ln staged N=%d ending=%s" % (N, ending))
    assert max_abs(u, fused) > 0.05, "x_ln was not taken"

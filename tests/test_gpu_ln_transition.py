"""GPU parity of the LayerNorm and transition kernels against the CPU oracle (same seeded inputs)."""
import pytest
import torch

from _util import assert_bf16_close, assert_bf16_residual_close, assert_f32_close
from oracle import stock as S

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _g(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("din,dout", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                      (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("rows,cols", [(1000, 128), (37, 256), (5, 384)])
def test_layer_norm(din, dout, rows, cols):
    from fpf_hip.kernels import ln
    g = _g(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 3 + 0.5).to(din)
    w = 1 + 0.1 * torch.randn(cols, generator=g)
    b = 0.1 * torch.randn(cols, generator=g)
    word = "fast" if din == torch.bfloat16 else "exact"
    y, sel = ln.layer_norm(x.to(DEV), (cols,), w.to(DEV), b.to(DEV), 1e-5, word=word, out_dtype=dout)
    torch.cuda.synchronize()
    ref = S.layer_norm(x.double(), w.double(), b.double(), 1e-5)
    if dout == torch.float32 and din == torch.float32:
        assert_f32_close(y, ref, "ln fp32")
    else:
        assert_bf16_close(y, ref, "ln")
    assert sel.row in ("hip_gfx950", "hip_gfx950_f32")


def _tr_weights(c, hidden, seed, dtype):
    g = _g(seed)
    wa = torch.randn(hidden, c, generator=g) / c ** 0.5
    wb = torch.randn(hidden, c, generator=g) / c ** 0.5
    wo = torch.randn(c, hidden, generator=g) / hidden ** 0.5
    lw = 1 + 0.1 * torch.randn(c, generator=g)
    lb = 0.1 * torch.randn(c, generator=g)
    return [t.to(dtype) for t in (wa, wb, wo)] + [lw, lb]


@pytest.mark.parametrize("rows", [4096, 1000, 1])
@pytest.mark.parametrize("residual,masked", [(False, False), (True, True)])
def test_transition_bf16(rows, residual, masked):
    from fpf_hip.kernels import transition as T
    c, hidden = 128, 512
    wa, wb, wo, lw, lb = _tr_weights(c, hidden, 11, torch.bfloat16)
    x = torch.randn(rows, c, generator=_g(rows)).to(torch.bfloat16)
    mask = (torch.rand(rows, generator=_g(3)) > 0.2).float() if masked else None
    W = T.pack(w_a=wa.to(DEV), w_b=wb.to(DEV), w_o=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV))
    y, sel = T.transition(x.to(DEV), W, word="fast", residual=residual, mask=None if mask is None else mask.to(DEV))
    torch.cuda.synchronize()
    assert sel.row == "hip_gfx950"
    ref = S.transition(x.float(), wa.float(), wb.float(), wo.float(), lw, lb, residual=residual, mask=mask, dtype=torch.float32)
    if residual:
        assert_bf16_residual_close(y, ref, "transition residual")
    else:
        assert_bf16_close(y, ref, "transition update")
    if masked:
        assert torch.equal(y.cpu()[mask == 0], x[mask == 0]), "masked rows must equal x bit for bit"


@pytest.mark.parametrize("hidden", [32, 64, 96, 256])
def test_transition_bf16_chunk_counts(hidden):
    """Hidden sizes of 1, 2, 3 and 8 weight chunks: the skewed early / late waves and the chunk ring's edges."""
    from fpf_hip.kernels import transition as T
    wa, wb, wo, lw, lb = _tr_weights(128, hidden, 13, torch.bfloat16)
    x = torch.randn(1000, 128, generator=_g(hidden)).to(torch.bfloat16)
    W = T.pack(w_a=wa.to(DEV), w_b=wb.to(DEV), w_o=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV))
    y, _ = T.transition(x.to(DEV), W, word="fast", residual=True)
    torch.cuda.synchronize()
    ref = S.transition(x.float(), wa.float(), wb.float(), wo.float(), lw, lb, residual=True, dtype=torch.float32)
    assert_bf16_residual_close(y, ref, "transition hidden %d" % hidden)


def test_transition_bf16_in_place_equals_out_of_place():
    from fpf_hip.kernels import transition as T
    wa, wb, wo, lw, lb = _tr_weights(128, 512, 12, torch.bfloat16)
    x = torch.randn(3000, 128, generator=_g(5)).to(torch.bfloat16).to(DEV)
    W = T.pack(w_a=wa.to(DEV), w_b=wb.to(DEV), w_o=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV))
    y1, _ = T.transition(x, W, word="fast", residual=True)
    x2 = x.clone()
    y2, _ = T.transition(x2, W, word="fast", residual=True, out=x2)
    torch.cuda.synchronize()
    assert y2.data_ptr() == x2.data_ptr()
    assert torch.equal(y1, x2)


@pytest.mark.parametrize("rows", [777, 4096])
def test_transition_fp32_exact(rows):
    from fpf_hip.kernels import transition as T
    c, hidden = 128, 512
    wa, wb, wo, lw, lb = _tr_weights(c, hidden, 13, torch.float32)
    x = torch.randn(rows, c, generator=_g(rows + 1))
    W = T.pack(w_a=wa.to(DEV), w_b=wb.to(DEV), w_o=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV))
    y, sel = T.transition(x.to(DEV), W, word="exact", residual=False)
    torch.cuda.synchronize()
    assert sel.row == "hip_gfx950_f32"
    ref = S.transition(x, wa, wb, wo, lw, lb, dtype=torch.float64)
    assert_f32_close(y, ref, "transition fp32")


@pytest.mark.parametrize("affine", [True, False])
def test_transition_fp32_exact_residual_mask(affine):
    """The fp32 matrix-core kernel (c = 128) with the residual, a row mask of arbitrary values and with / without the
    LayerNorm affine, hidden 256 (8 chunks); a ragged last tile (1000 rows)."""
    from fpf_hip.kernels import transition as T
    c, hidden, rows = 128, 256, 1000
    wa, wb, wo, lw, lb = _tr_weights(c, hidden, 14, torch.float32)
    if not affine:
        lw = lb = None
    x = torch.randn(rows, c, generator=_g(3))
    m = torch.rand(rows, generator=_g(4)) * (torch.rand(rows, generator=_g(5)) > 0.2).float()
    W = T.pack(w_a=wa.to(DEV), w_b=wb.to(DEV), w_o=wo.to(DEV), ln_w=None if lw is None else lw.to(DEV), ln_b=None if lb is None else lb.to(DEV))
    y, sel = T.transition(x.to(DEV), W, word="exact", residual=True, mask=m.to(DEV))
    torch.cuda.synchronize()
    assert sel.row == "hip_gfx950_f32"
    upd = S.transition(x, wa, wb, wo, lw, lb, dtype=torch.float64)
    assert_f32_close(y, x.double() + m.double()[:, None] * upd, "transition fp32 residual mask affine=%s" % affine)


# ------------------------------------------------------------------------------------------------ the block-glue transition face
@pytest.mark.parametrize("split", [("a", "b"), ("b", "a")])
def test_pair_fused_transition_face(split):
    """pair_fused.transition over pack_transition_weights (common/opt_core/opt_core/attn/pair_fused.py:1519-1585, :744-780) on a
    pair tensor [1, 96, 96, 128]: the fused w_ab in both ab_split orders (rows of each half named by the split), a per-position mask
    with zero and fractional values, the residual, and in place (out = x).  Against the fp32 statement at the bf16 bars (the
    residual form with the half-ulp allowance), masked positions equal to x bit for bit, and in place equal to out of place."""
    from fpf_hip.attn import pair_fused as PF
    c, hidden, n = 128, 512, 96
    wa, wb, wo, lw, lb = _tr_weights(c, hidden, 21, torch.bfloat16)
    halves = {"a": wa, "b": wb}
    w_ab = torch.cat([halves[split[0]], halves[split[1]]], 0).to(DEV)
    T = PF.pack_transition_weights(w_out=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV), w_ab=w_ab, ab_split=split)
    assert (T.C, T.NH, T.n) == (c, hidden, 4)
    x = torch.randn(1, n, n, c, generator=_g(22)).to(torch.bfloat16)
    m = (torch.rand(1, n, n, generator=_g(23)) > 0.2).float()
    m[0, 3, :] = 0.5
    print("[C3] pair_fused.transition split=%s" % (split,), flush=True)
    xd, md = x.to(DEV), m.to(DEV)
    y = PF.transition(xd, T, residual=True, mask=md)
    xi = xd.clone()
    yi = PF.transition(xi, T, residual=True, mask=md, out=xi)
    u = PF.transition(xd, T, residual=False)
    torch.cuda.synchronize()
    assert yi.data_ptr() == xi.data_ptr() and torch.equal(yi, y), "in place != out of place"
    assert torch.equal(xd.cpu(), x), "out of place must leave x untouched"
    ref_u = S.transition(x.float(), wa.float(), wb.float(), wo.float(), lw, lb, dtype=torch.float32)
    assert_bf16_close(u, ref_u, "C3 update split=%s" % (split,))
    ref = S.transition(x.float(), wa.float(), wb.float(), wo.float(), lw, lb, residual=True, mask=m, dtype=torch.float32)
    assert_bf16_residual_close(y, ref, "C3 residual + mask split=%s" % (split,))
    assert torch.equal(y.cpu()[m == 0], x[m == 0]), "masked positions must equal x bit for bit"


def test_pair_fused_transition_face_matches_the_kernel_face():
    """The glue face and kernels.transition.transition run the same kernel on the same pack: bitwise the same result, both ab_split
    orders naming the same halves included."""
    from fpf_hip.attn import pair_fused as PF
    from fpf_hip.kernels import transition as TRK
    wa, wb, wo, lw, lb = _tr_weights(128, 512, 24, torch.bfloat16)
    x = torch.randn(1, 64, 64, 128, generator=_g(25)).to(torch.bfloat16).to(DEV)
    T1 = PF.pack_transition_weights(w_out=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV), w_a=wa.to(DEV), w_b=wb.to(DEV))
    T2 = PF.pack_transition_weights(w_out=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV), w_ab=torch.cat([wb, wa], 0).to(DEV), ab_split=("b", "a"))
    K = TRK.pack(w_a=wa.to(DEV), w_b=wb.to(DEV), w_o=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV))
    y1 = PF.transition(x, T1, residual=True)
    y2 = PF.transition(x, T2, residual=True)
    y3, _ = TRK.transition(x, K, word="fast", residual=True)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(y1, y3)


@pytest.mark.parametrize("residual", [False, True])
def test_transition_bf16_x_ln(residual):
    """The caller's own LayerNorm output x_ln (pair_fused.py:1089-1094, ln="stock"; kernels.transition's x_ln) is projected in place
    of the in-kernel LayerNorm and the residual adds x: x_ln = bf16(LN(x) * 1.05 + 0.02), against the statement with that x_ln,
    through both faces, in place as well."""
    from fpf_hip.attn import pair_fused as PF
    from fpf_hip.kernels import transition as T
    wa, wb, wo, lw, lb = _tr_weights(128, 512, 31, torch.bfloat16)
    x = torch.randn(1, 40, 50, 128, generator=_g(32)).to(torch.bfloat16)
    xl = (S.layer_norm(x.float(), lw, lb, 1e-5) * 1.05 + 0.02).to(torch.bfloat16).contiguous()
    W = T.pack(w_a=wa.to(DEV), w_b=wb.to(DEV), w_o=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV))
    TW = PF.pack_transition_weights(w_out=wo.to(DEV), ln_w=lw.to(DEV), ln_b=lb.to(DEV), w_a=wa.to(DEV), w_b=wb.to(DEV))
    xd, xld = x.to(DEV), xl.to(DEV)
    print("[x_ln] transition residual=%s" % residual, flush=True)
    y, sel = T.transition(xd, W, word="fast", residual=residual, x_ln=xld)
    y2 = PF.transition(xd, TW, residual=residual, ln="stock", x_ln=xld)
    xi = xd.clone()
    y3 = PF.transition(xi, TW, residual=residual, ln="stock", x_ln=xld, out=xi)
    plain, _ = T.transition(xd, W, word="fast", residual=residual)
    torch.cuda.synchronize()
    assert sel.row == "hip_gfx950"
    assert torch.equal(y, y2) and torch.equal(y, y3)
    ref = S.transition(x.float(), wa.float(), wb.float(), wo.float(), lw, lb, residual=residual, dtype=torch.float32, x_ln=xl.float())
    (assert_bf16_residual_close if residual else assert_bf16_close)(y, ref, "transition x_ln residual=%s" % residual)
    assert (y.float() - plain.float()).abs().max().item() > 0.05, "x_ln was not taken"

"""GPU parity of the triangle-multiplication kernels (K1 -> contraction -> K3) against the CPU oracle."""
import json
import os

import pytest
import torch

from _util import assert_bf16_close, assert_bf16_residual_close, assert_bf16_ulp_close, assert_f32_close, max_abs, rel_l2
from conftest import GOLDEN
from oracle import stock as S
from oracle import vectors as V

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _weights(c, seed, dtype, ln_affine=True):
    g = torch.Generator().manual_seed(seed)
    w = {k: torch.randn(c, c, generator=g) / c ** 0.5 for k in ("w_ag", "w_ap", "w_bg", "w_bp", "w_o", "w_og")}
    if ln_affine:
        w.update(ln_in_w=1 + 0.1 * torch.randn(c, generator=g), ln_in_b=0.1 * torch.randn(c, generator=g),
                 ln_out_w=1 + 0.1 * torch.randn(c, generator=g), ln_out_b=0.1 * torch.randn(c, generator=g))
    else:
        w.update(ln_in_w=torch.ones(c), ln_in_b=torch.zeros(c), ln_out_w=torch.ones(c), ln_out_b=torch.zeros(c))
    return {k: (v.to(dtype) if k.startswith("w_") else v) for k, v in w.items()}


def _dev(w):
    return {k: v.to(DEV) for k, v in w.items()}


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("B,N,masked", [(1, 64, False), (1, 100, True), (2, 37, True)])
def test_trimul_bf16(direction, B, N, masked):
    from fpf_hip.kernels import trimul as TM
    w = _weights(128, 1, torch.bfloat16)
    g = torch.Generator().manual_seed(N)
    z = torch.randn(B, N, N, 128, generator=g).to(torch.bfloat16)
    mask = None
    if masked:
        mask = torch.ones(B, N, N)
        mask[:, N - 5:, :] = 0
        mask[:, :, N - 5:] = 0
    out = TM.triangle_multiplication(z.to(DEV), None if mask is None else mask.to(DEV), direction=direction, weights=_dev(w), word="fast")
    torch.cuda.synchronize()
    ref = S.trimul(z.float(), mask, direction=direction, weights={k: v.float() for k, v in w.items()}, dtype=torch.float32)
    assert_bf16_close(out, ref, "trimul %s B%d N%d" % (direction, B, N))


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("N", [512, 768, 800, 600])
def test_trimul_bf16_256_tiles_sampled_rows(direction, N):
    """The persistent 256 x 256 contraction, whose slab ring runs across tile boundaries (N = 512: two tiles per workgroup;
    N = 768, the bench shape: four or five), also on planes padded to an odd multiple of 128 (N = 800 -> 896, N = 600 -> 640),
    whose last tile row and column are half inside the plane.  Sampled rows on both sides of every tile boundary against the
    fp32 oracle, with a ragged mask, at the bf16 bars with max-abs counted above the output's half-ulp (these updates reach
    |value| of a few units, where a bf16 output's own rounding is up to 1.6e-2: the max-abs measures 1.6-2.0e-2 at every N, with
    rel-L2 4.4-4.5e-3); a second call is bitwise the first."""
    from fpf_hip.kernels import trimul as TM
    w = _weights(128, 11, torch.bfloat16)
    g = torch.Generator().manual_seed(N + 1)
    z = torch.randn(N, N, 128, generator=g).to(torch.bfloat16)
    mask = torch.ones(N, N)
    mask[N - 7:, :] = 0
    mask[:, N - 7:] = 0
    print("[trimul256] %s N=%d" % (direction, N), flush=True)
    zd, md, wd = z.to(DEV), mask.to(DEV), _dev(w)
    u1 = TM.triangle_multiplication(zd, md, direction=direction, weights=wd, word="fast")
    u2 = TM.triangle_multiplication(zd, md, direction=direction, weights=wd, word="fast")
    torch.cuda.synchronize()
    assert torch.equal(u1, u2)
    rows = sorted(set([0, 1, 130, 255, 256, 383, N // 2 + 3, N - 256, N - 130, N - 8, N - 1]))
    got = u1[rows].cpu()
    ref = S.trimul_rows(z.float(), mask, rows, direction=direction, weights={k: v.float() for k, v in w.items()}, dtype=torch.float32)
    assert_bf16_ulp_close(got, ref, "trimul256 %s N%d rows %s" % (direction, N, rows))


def test_trimul_bf16_residual_in_place_equals_out_of_place():
    from fpf_hip.kernels import trimul as TM
    w = _dev(_weights(128, 2, torch.bfloat16))
    z = torch.randn(1, 96, 96, 128, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    y1 = TM.triangle_multiplication(z, None, direction="incoming", weights=w, word="fast", residual=True)
    z2 = z.clone()
    y2 = TM.triangle_multiplication(z2, None, direction="incoming", weights=w, word="fast", residual=True, out=z2)
    torch.cuda.synchronize()
    assert y2.data_ptr() == z2.data_ptr() and torch.equal(y1, z2)


def test_trimul_bf16_zero_mask_zero_ln_out_bias_gives_exact_zero():
    from fpf_hip.kernels import trimul as TM
    w = _weights(128, 4, torch.bfloat16)
    w["ln_out_b"] = torch.zeros(128)
    z = torch.randn(50, 50, 128, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    out = TM.triangle_multiplication(z.to(DEV), torch.zeros(50, 50, device=DEV), direction="outgoing", weights=_dev(w), word="fast")
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0


def test_trimul_bf16_masked_rows_update_is_gate_times_bias_projection():
    """A pixel whose row AND column are masked sees X = 0 for every k, so its update is sigmoid(x W_og) (ln_out_b W_o^T)."""
    from fpf_hip.kernels import trimul as TM
    w = _weights(128, 6, torch.bfloat16)
    w["ln_out_b"] = torch.zeros(128)
    N = 40
    z = torch.randn(N, N, 128, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    mask = torch.ones(N, N)
    mask[N - 3:, :] = 0
    mask[:, N - 3:] = 0
    out = TM.triangle_multiplication(z.to(DEV), mask.to(DEV), direction="outgoing", weights=_dev(w), word="fast").cpu()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[N - 3:, N - 3:]) == 0          # X = 0 there and beta_out = 0 -> exactly 0


TRIMUL = json.load(open(os.path.join(GOLDEN, "trimul_cases.json")))["cases"]
CF = [c for c in TRIMUL if c["form"] == "bf16" and c["c_z"] == 128]          # N 32 .. 403 (the ragged incoming N = 403 included)


@pytest.mark.parametrize("case", CF, ids=[c["id"] for c in CF])
def test_trimul_closed_form_vectors(case):
    """The reference's closed-form cases: error vs the fp64 statement within the BASELINE bars, reported beside the H100
    kernel's recorded error for the same inputs."""
    from fpf_hip.kernels import trimul as TM
    z, mask, w = V.trimul_inputs(case)
    print("[case] %s" % case["id"], flush=True)
    out = TM.triangle_multiplication(z.to(DEV), None if mask is None else mask.to(DEV), direction=case["direction"], weights=_dev(w),
                                     word="fast", residual=case["residual"])
    torch.cuda.synchronize()
    ref = S.trimul(z, mask, direction=case["direction"], weights=w, residual=case["residual"], dtype=torch.float64)
    (assert_bf16_residual_close if case["residual"] else assert_bf16_close)(out, ref, case["id"])
    h100 = case["expected"].get("sm90", {}).get("numerics", {})
    print("[parity] %s ours max_abs=%.3e rel_rms=%.3e | H100 native max_abs=%s rel_rms=%s" % (
        case["id"], max_abs(out, ref), rel_l2(out, ref), h100.get("max_abs_fp64"), h100.get("rel_rms_fp64")))


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("N,masked", [(48, False), (70, True)])
def test_trimul_fp32_exact(direction, N, masked):
    from fpf_hip.kernels import trimul as TM
    w = _weights(128, 8, torch.float32)
    z = torch.randn(N, N, 128, generator=torch.Generator().manual_seed(N))
    mask = None
    if masked:
        mask = torch.ones(N, N)
        mask[N - 4:, :] = 0
    out = TM.triangle_multiplication(z.to(DEV), None if mask is None else mask.to(DEV), direction=direction, weights=_dev(w), word="hip_gfx950_f32")
    torch.cuda.synchronize()
    ref = S.trimul(z, mask, direction=direction, weights=w, dtype=torch.float64)
    assert_f32_close(out, ref, "trimul fp32 %s N%d" % (direction, N))


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_fp32_exact_batch_residual_ragged(direction):
    """The fp32 matrix-core kernels past one contraction tile: batch 2, N = 300 (planes of 384: 3 x 3 tiles of 128, the last
    one ragged), residual, a mask with padded tail rows / columns and random holes."""
    from fpf_hip.kernels import trimul as TM
    N = 300
    w = _weights(128, 9, torch.float32)
    g = torch.Generator().manual_seed(11)
    z = torch.randn(2, N, N, 128, generator=g)
    valid = torch.ones(N)
    valid[N - 7:] = 0
    mask = torch.outer(valid, valid).expand(2, N, N) * (torch.rand(2, N, N, generator=g) > 0.05).float()
    print("[case] trimul fp32 %s B=2 N=%d residual" % (direction, N), flush=True)
    out = TM.triangle_multiplication(z.to(DEV), mask.to(DEV), direction=direction, weights=_dev(w), word="hip_gfx950_f32", residual=True)
    torch.cuda.synchronize()
    ref = S.trimul(z, mask, direction=direction, weights=w, residual=True, dtype=torch.float64)
    assert_f32_close(out, ref, "trimul fp32 %s B2 N%d residual" % (direction, N))


# ---------------------------------------------------------------------------------------------------------- the f32z_bf16 class
def test_trimul_f32z_reference_case_under_autocast():
    """The reference-held case c128x128_n400_out_f32z_res1_mnone_fast (tests/golden/trimul_cases.json): an fp32 z and fp32
    weights under bf16 autocast -- the f32z_bf16 class, served by the bf16 row with fp32 z / out -- against the fp64
    statement, next to the reference's recorded numbers for its fast row."""
    from fpf_hip.kernels import trimul as TM
    case = [c for c in TRIMUL if c["id"] == "c128x128_n400_out_f32z_res1_mnone_fast"][0]
    z, mask, w = V.trimul_inputs(case)
    assert z.dtype == torch.float32 and mask is None
    print("[case] %s" % case["id"], flush=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = TM.triangle_multiplication(z.to(DEV), None, direction=case["direction"], weights=_dev(w), word="fast", residual=True)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    ref = S.trimul(z, None, direction=case["direction"], weights=w, residual=True, dtype=torch.float64)
    assert_bf16_close(out, ref, case["id"])
    rec = case["expected"]["sm80"]["numerics"]
    print("[parity] %s ours max_abs=%.3e rel_rms=%.3e | reference fast row (sm80) max_abs=%.3e rel_rms=%.3e" % (
        case["id"], max_abs(out, ref), rel_l2(out, ref), rec["max_abs_fp64"], rec["rel_rms_fp64"]))


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_f32z_update_is_the_bf16_update_of_the_rounded_z(direction):
    """The f32z_bf16 kernels read z rounded once to bf16 (the reference's compute_input): their fp32 update, rounded to bf16,
    is the bf16 row's update on z.to(bfloat16) bit for bit; the residual form adds the fp32 z.  Ragged mask, N = 300."""
    from fpf_hip.kernels import trimul as TM
    N = 300
    w = _weights(128, 21, torch.bfloat16)
    g = torch.Generator().manual_seed(22)
    z = torch.randn(N, N, 128, generator=g).to(DEV)
    mask = torch.ones(N, N)
    mask[N - 5:, :] = 0
    mask = mask.to(DEV)
    sel = TM.select((9, 5), "bf16", 128, 128, N, direction, word="fast", residency="fp32")
    u32 = TM.triangle_multiplication(z, mask, direction=direction, weights=_dev(w), selection=sel)
    u16 = TM.triangle_multiplication(z.to(torch.bfloat16), mask, direction=direction, weights=_dev(w), word="fast")
    r32 = TM.triangle_multiplication(z, mask, direction=direction, weights=_dev(w), selection=sel, residual=True)
    torch.cuda.synchronize()
    assert u32.dtype == torch.float32 and u16.dtype == torch.bfloat16
    assert torch.equal(u32.to(torch.bfloat16), u16)
    assert torch.equal(r32, z + u32)


def test_trimul_fp32_narrow_channels_scalar_path():
    """c_z = c_h = 64 is served by the scalar fp32 kernels (the matrix-core form is built for 128)."""
    from fpf_hip.kernels import trimul as TM
    N = 40
    w = _weights(64, 10, torch.float32)
    z = torch.randn(N, N, 64, generator=torch.Generator().manual_seed(12))
    out = TM.triangle_multiplication(z.to(DEV), None, direction="incoming", weights=_dev(w), word="hip_gfx950_f32", residual=True)
    torch.cuda.synchronize()
    ref = S.trimul(z, None, direction="incoming", weights=w, residual=True, dtype=torch.float64)
    assert_f32_close(out, ref, "trimul fp32 c64")


@pytest.mark.parametrize("N", [800, 600])
def test_trimul_half_inside_tiles_repeat_bitwise(N):
    """Planes padded to an odd multiple of 128 (N = 800 -> 896, N = 600 -> 640) end half way into the contraction's 256-row
    tiles: the waves whose quarter of such a tile is a duplicate store nothing, and their next tile's slab waits must not
    count stores they never issued.  20 calls in a row on one input, both directions, with a mask: all finite and bitwise
    equal to the first."""
    from fpf_hip.kernels import trimul as TM
    g = torch.Generator().manual_seed(N + 3)
    w = _dev(_weights(128, 5, torch.bfloat16))
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16).to(DEV)
    mask = (torch.rand(1, N, N, generator=g) > 0.2).float().to(DEV)
    for d in ("outgoing", "incoming"):
        print("[trimul] half-inside tiles N=%d %s x 20" % (N, d), flush=True)
        cache = {}
        first = TM.triangle_multiplication(z, mask, direction=d, weights=w, word="fast", cache=cache)
        torch.cuda.synchronize()
        assert torch.isfinite(first.float()).all()
        for rep in range(1, 20):
            out = TM.triangle_multiplication(z, mask, direction=d, weights=w, word="fast", cache=cache)
            assert torch.equal(out, first), "%s run %d differs from run 0" % (d, rep)

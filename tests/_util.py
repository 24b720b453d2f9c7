"""Shared helpers of the parity tests (error metrics with the BASELINE tolerances)."""
import torch

BF16_MAX_ABS = 2e-2      # bf16 fast tier vs the fp32 reference
BF16_REL_L2 = 5e-3
F32_REL = 1e-5           # fp32 exact tier vs the fp32 reference


def rel_l2(out, ref):
    o, r = out.double().cpu(), ref.double().cpu()
    return ((o - r).norm() / r.norm().clamp_min(1e-30)).item()


def max_abs(out, ref):
    return (out.double().cpu() - ref.double().cpu()).abs().max().item()


def assert_bf16_close(out, ref, what=""):
    ma, rl = max_abs(out, ref), rel_l2(out, ref)
    print("[parity] %s max_abs=%.3e rel_l2=%.3e" % (what, ma, rl))
    assert ma <= BF16_MAX_ABS and rl <= BF16_REL_L2, "%s max_abs=%.3e rel_l2=%.3e" % (what, ma, rl)
    return ma, rl


def assert_f32_close(out, ref, what=""):
    rl = rel_l2(out, ref)
    print("[parity] %s rel_l2=%.3e" % (what, rl))
    assert rl <= F32_REL, "%s rel_l2=%.3e" % (what, rl)
    return rl


def assert_bf16_ulp_close(out, ref, what=""):
    """bf16 outputs whose magnitude reaches 4 and beyond (residual forms z + update, large updates): the bars applied to the
    error in excess of the half-ulp of the bf16 output itself, which no kernel with a bf16 output can avoid once |value| >= 4
    (half-ulp 2^-7 there, 2^-6 from 8).  The relative-L2 bar is unchanged."""
    o, r = out.double().cpu(), ref.double().cpu()
    ulp = torch.pow(2.0, torch.floor(torch.log2(r.abs().clamp_min(2.0 ** -126))) - 7)
    excess = ((o - r).abs() - 0.5 * ulp).max().item()
    rl = rel_l2(o, r)
    print("[parity] %s max_abs=%.3e max(|err| - ulp/2)=%.3e rel_l2=%.3e" % (what, max_abs(o, r), excess, rl))
    assert excess <= BF16_MAX_ABS and rl <= BF16_REL_L2, "%s excess=%.3e rel_l2=%.3e" % (what, excess, rl)
    return excess, rl


assert_bf16_residual_close = assert_bf16_ulp_close


SAME_CLASS_RMS = 1.25    # common/opt_core/opt_core/kernels/fpf_trimul_v4/generic.py:42-43: a bf16 kernel is admitted when its error
SAME_CLASS_MAX = 2.5     # is at most 1.25x (rms) and 2.5x (max-abs) the bf16-autocast torch statement's own error


def assert_same_class(out, ref, yardstick, what=""):
    """Block-level numerics: ``out``'s error vs the fp32 statement ``ref`` within the SAME_CLASS multiples of the bf16-autocast
    statement's own error (``yardstick``, oracle.stock.*_autocast on the same inputs).  A multi-site bf16 block cannot meet the
    per-op absolute bars (the autocast statement itself exceeds them), so the block is held to the class its kit admits;
    the absolute numbers are printed beside the ratios."""
    ma, rl = max_abs(out, ref), rel_l2(out, ref)
    ya, yr = max_abs(yardstick, ref), rel_l2(yardstick, ref)
    print("[same-class] %s ours max_abs=%.3e rel_l2=%.3e | autocast statement max_abs=%.3e rel_l2=%.3e | ratio rms %.3f max %.3f "
          "(bars %.2f / %.2f; absolute bars %s)" % (what, ma, rl, ya, yr, rl / yr, ma / ya, SAME_CLASS_RMS, SAME_CLASS_MAX,
                                                    "met" if ma <= BF16_MAX_ABS and rl <= BF16_REL_L2 else "not met"))
    assert rl <= SAME_CLASS_RMS * yr and ma <= SAME_CLASS_MAX * ya, "%s: rms x%.3f max x%.3f of the autocast statement" % (what, rl / yr, ma / ya)
    return rl / yr, ma / ya

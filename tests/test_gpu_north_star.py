"""The north-star workload itself -- the Pairformer pair stack at N = 768, c_z = 128, bf16, in place on one resident z
(boltz2/stock/src/boltz/model/layers/pairformer.py:75-102 per block; the resident-z composition of
boltz2/opt/forward/pairfuse/bz_pairfuse.py:747-774) -- checked at its own size:

  * two stacked blocks against the fp32 statements, held to the reference's SAME_CLASS multiples of the bf16-autocast statement
    (common/opt_core/opt_core/kernels/fpf_trimul_v4/generic.py:42-43), as the N = 48 / 96 blocks are;
  * every site of one block, fed the same bf16 input, against its fp32 statement: the absolute bars where the site's own
    rounding allows them, and the per-site margins printed;
  * the 48-block stack: finite everywhere and bitwise identical from run to run;
  * one masked block repeated 20 times bitwise (the persistent 8-wave triangle-attention core, both nodes, with its keep table).

At N = 768 the CPU takes minutes per fp32 block, so the statements (oracle.stock, pinned on the CPU by tests/test_oracle.py) are
evaluated here on the GPU in fp32 with TF32 off: plain torch matmul / softmax / einsum on device tensors, the same code.
"""
import pytest
import torch

from _util import BF16_MAX_ABS, BF16_REL_L2, assert_same_class, max_abs, rel_l2
from oracle import stock as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
N = 768


def _bf16_weights(params):
    """bf16-representable projection weights, so the statements and the bf16 kernels see the same values."""
    for site in ("tmo", "tmi", "tas", "tae", "tr"):
        for k_, v_ in params[site].items():
            if hasattr(v_, "dtype") and not k_.startswith("ln_"):
                params[site][k_] = v_.to(torch.bfloat16).float()
    return params


def _on_device(params):
    return {site: {k_: (v_.to(DEV) if hasattr(v_, "to") else v_) for k_, v_ in p.items()} for site, p in params.items()}


@pytest.fixture(autouse=True)
def _fp32_matmul():
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = prev


def test_two_block_stack_n768_same_class():
    """Two stacked pair blocks at the metric's shape (mask all ones, seed-fixed weights per block) against the fp32 statements of
    both blocks, within SAME_CLASS of the two-block bf16-autocast statement (whose residual stream stays fp32)."""
    from fpf_hip import pairformer as PFM
    params = [_bf16_weights(PFM.random_params(seed=100 + l)) for l in range(2)]
    blocks = [PFM.PairBlock(p, DEV, torch.bfloat16) for p in params]
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    mask = torch.ones(1, N, N, device=DEV)
    print("[north-star] 2-block stack N=%d" % N, flush=True)
    zd = z.to(DEV)
    PFM.pair_stack(zd, mask, blocks)
    torch.cuda.synchronize()
    assert torch.isfinite(zd.float()).all()
    ref, ys = z.to(DEV).float(), z.to(DEV).float()
    for p in params:
        pd = _on_device(p)
        ref = S.pair_block(ref, mask, pd, dtype=torch.float32)
        ys = S.pair_block_autocast(ys, mask, pd)
    torch.cuda.synchronize()
    assert_same_class(zd.float(), ref, ys, "2-block stack N=%d" % N)


def test_pair_block_per_site_margins_n768():
    """Each site of one block at N = 768 (a ragged token mask: 740 live residues, 28 padded), fed the same bf16 input -- the fp32
    chain's state rounded to bf16 -- against the fp32 statement of that site: rel-L2 within the 5e-3 bar at every site; max-abs
    within 2e-2 for the triangle-attention sites (whose updates stay small) and SAME_CLASS for every site.  The printed lines are
    the per-site margins at the metric's size."""
    from fpf_hip import pairformer as PFM
    from fpf_hip.attn import pair_fused as PF
    from fpf_hip.kernels import transition as TR
    from fpf_hip.kernels import trimul as TM
    params = _bf16_weights(PFM.random_params(seed=7))
    pd = _on_device(params)
    blk = PFM.PairBlock(params, DEV, torch.bfloat16)
    valid = (torch.arange(N, device=DEV) < N - 28).float()
    mask = (valid[:, None] * valid[None, :]).unsqueeze(0)
    t = pd["tr"]
    sites = [
        ("trimul_out", lambda x: S.trimul(x, mask, direction="outgoing", weights=pd["tmo"], dtype=torch.float32),
         lambda x: S.trimul_autocast(x, mask, direction="outgoing", weights=pd["tmo"]),
         lambda xd: TM.triangle_multiplication(xd, mask, direction="outgoing", weights=blk.tmo, word="fast", cache=blk.cache_o)),
        ("trimul_in", lambda x: S.trimul(x, mask, direction="incoming", weights=pd["tmi"], dtype=torch.float32),
         lambda x: S.trimul_autocast(x, mask, direction="incoming", weights=pd["tmi"]),
         lambda xd: TM.triangle_multiplication(xd, mask, direction="incoming", weights=blk.tmi, word="fast", cache=blk.cache_i)),
        ("tri_att_start", lambda x: S.tri_attn(x, pd["tas"], mask, ending=False, dtype=torch.float32),
         lambda x: S.tri_attn_autocast(x, pd["tas"], mask, ending=False),
         lambda xd: PF.tri_attn_block(xd, blk.ta["tas"], mask, ending=False)),
        ("tri_att_end", lambda x: S.tri_attn(x, pd["tae"], mask, ending=True, dtype=torch.float32),
         lambda x: S.tri_attn_autocast(x, pd["tae"], mask, ending=True),
         lambda xd: PF.tri_attn_block(xd, blk.ta["tae"], mask, ending=True)),
        ("transition", lambda x: S.transition(x, t["w_a"], t["w_b"], t["w_o"], t["ln_w"], t["ln_b"], dtype=torch.float32),
         lambda x: S.transition_autocast(x, t["w_a"], t["w_b"], t["w_o"], t["ln_w"], t["ln_b"]),
         lambda xd: TR.transition(xd, blk.tr, word="fast")[0]),
    ]
    x32 = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).float().to(DEV)
    for name, f32, ac, hip in sites:
        xin = x32.to(torch.bfloat16)
        print("[north-star] site %s N=%d" % (name, N), flush=True)
        u = hip(xin.clone())
        ref = f32(xin.float())
        torch.cuda.synchronize()
        ma, rl = max_abs(u, ref), rel_l2(u, ref)
        print("[margin] site %s N=%d max_abs=%.3e rel_l2=%.3e (rel-L2 margin %.1f %% of the 5e-3 bar)"
              % (name, N, ma, rl, 100.0 * (1.0 - rl / BF16_REL_L2)), flush=True)
        assert rl <= BF16_REL_L2, "site %s rel_l2=%.3e" % (name, rl)
        if name.startswith("tri_att"):
            assert ma <= BF16_MAX_ABS, "site %s max_abs=%.3e" % (name, ma)
        assert_same_class(u.float(), ref, ac(xin.float()), "site %s N=%d" % (name, N))
        x32 = x32 + ref
        del u, ref


def test_stack_48_blocks_n768_finite_and_repeatable():
    """The north-star stack as bench.py times it (48 blocks, seeds 100 + l, z ~ N(0, 1) seed 5, mask all ones): every value finite
    after 48 in-place blocks, and a second pass from the same input bitwise equal to the first."""
    from fpf_hip import pairformer as PFM
    blocks = [PFM.PairBlock(PFM.random_params(seed=100 + l), DEV, torch.bfloat16) for l in range(48)]
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    mask = torch.ones(1, N, N, device=DEV)
    runs = []
    for rep in range(2):
        print("[north-star] 48-block stack pass %d" % rep, flush=True)
        zr = z.clone()
        PFM.pair_stack(zr, mask, blocks)
        runs.append(zr)
    torch.cuda.synchronize()
    assert torch.isfinite(runs[0].float()).all(), "non-finite values after 48 blocks"
    assert not torch.equal(runs[0], z)
    assert torch.equal(runs[0], runs[1]), "48-block stack differs between passes"


def test_pair_block_n768_masked_repeats_bitwise():
    """One block at N = 768 with an asymmetric random mask (keep tables on both triangle-attention nodes, masked trimul operands), 20
    calls on clones of one input: all finite and bitwise equal to the first.  The whole triangle-attention sites run the persistent
    8-wave core, whose DMA ring and bias buffers carry across work items."""
    from fpf_hip import pairformer as PFM
    blk = PFM.PairBlock(PFM.random_params(seed=9), DEV, torch.bfloat16)
    g = torch.Generator().manual_seed(10)
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16).to(DEV)
    mask = (torch.rand(1, N, N, generator=g) > 0.25).float().to(DEV)
    print("[north-star] masked block x 20", flush=True)
    first = z.clone()
    PFM.pair_block(first, mask, blk)
    torch.cuda.synchronize()
    assert torch.isfinite(first.float()).all()
    for rep in range(1, 20):
        zr = z.clone()
        PFM.pair_block(zr, mask, blk)
        assert torch.equal(zr, first), "run %d differs from run 0" % rep

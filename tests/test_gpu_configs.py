"""The BASELINE configs against the CPU oracle at their own sizes, the projection biases, and the layer's run contract
(bitwise repeatability, no host synchronisation after the first call).

    configs[0]  the fp32 pair block, N = 64, through the exact row hip_gfx950_f32: rel-L2 <= 1e-5 vs the fp64 statements
    configs[1]  triangle attention, N = 384, the last 38 residues masked on both axes, both nodes: bf16 bars vs fp32; rows whose
                keys are all masked are the uniform mean
    configs[2]  triangle multiplication at N = 768: tests/test_gpu_trimul.py (sampled rows of both directions)
    configs[3]  one Pairformer layer at N = 512 (pair track bf16, single track fp32) vs the fp32 statements, held to the
                reference's SAME_CLASS multiples of the bf16-autocast statement's error
    metric      the tri-att block at N = 768 (the 8-wave block-layout core) on sampled rows, asymmetric mask, both nodes
"""
import pytest
import torch

from _util import assert_bf16_close, assert_f32_close, assert_same_class, max_abs, rel_l2
from oracle import stock as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _bf16_weights(params):
    """bf16-representable projection weights, so the oracle and the bf16 kernels see the same values."""
    for site in ("tmo", "tmi", "tas", "tae", "tr"):
        for k_, v_ in params[site].items():
            if hasattr(v_, "dtype") and not k_.startswith("ln_"):
                params[site][k_] = v_.to(torch.bfloat16).float()
    return params


def _ta_weights(seed, biases=False):
    P = S.make_block_params(c_z=128, heads=4, head_dim=32, seed=seed)["tas"]
    g = torch.Generator().manual_seed(seed + 100)
    P["ln_w"] = 1 + 0.1 * torch.randn(128, generator=g)
    P["ln_b"] = 0.1 * torch.randn(128, generator=g)
    if biases:
        P["b_g"] = torch.randn(128, generator=g)
        P["b_o"] = 0.2 * torch.randn(128, generator=g)
    for n in ("w_q", "w_k", "w_v", "w_g", "w_b", "w_o", "b_g", "b_o"):
        if n in P:
            P[n] = P[n].to(torch.bfloat16).float()
    return P


def _ta_pack(P, dtype=torch.bfloat16):
    from fpf_hip.attn import pair_fused as PF
    d = {n: P[n].to(DEV, dtype) for n in ("w_q", "w_k", "w_v", "w_g", "w_b", "w_o")}
    return PF.pack_triattn_weights(n_heads=4, head_dim=32, ln_w=P["ln_w"].to(DEV), ln_b=P["ln_b"].to(DEV),
                                   b_g=P.get("b_g"), b_o=P.get("b_o"), **d)


# ------------------------------------------------------------------------------------------------------------------ configs[0]
def test_config0_fp32_block_through_the_exact_row():
    """one pair block at N = 64, c_z = 128, 4 x 32 heads, transition 4x, fp32, z ~ N(0, 1) and weights
    N(0, 1/fan_in) from seed 0 (module order), LN 1 / 0, mask all ones -- every site on row hip_gfx950_f32."""
    from fpf_hip import pairformer as PFM
    params = S.make_block_params(c_z=128, heads=4, head_dim=32, seed=0)
    z = torch.randn(1, 64, 64, 128, generator=torch.Generator().manual_seed(0))
    mask = torch.ones(1, 64, 64)
    blk = PFM.PairBlock(params, DEV, torch.float32)
    zd = z.to(DEV)
    print("[config0] fp32 block N=64 row hip_gfx950_f32", flush=True)
    PFM.pair_block(zd, mask.to(DEV), blk, word="hip_gfx950_f32")
    torch.cuda.synchronize()
    ref = S.pair_block(z.double(), mask, params, dtype=torch.float64)
    assert_f32_close(zd, ref, "config0 fp32 block")


# ------------------------------------------------------------------------------------------------------------------ configs[1]
@pytest.mark.parametrize("ending", [False, True])
def test_config1_tri_attn_n384_padded(ending):
    """N = 384, pair mask m[i, j] = (i < 346) & (j < 346).  Attention rows >= 346 have no live key: their
    update is W_o (sigmoid(g) * mean_k v) + the same over every key, checked against that closed form as well as the statement."""
    from fpf_hip.attn import pair_fused as PF
    N, L = 384, 346
    P = _ta_weights(11)
    W = _ta_pack(P)
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    valid = (torch.arange(N) < L).float()
    mask = torch.outer(valid, valid).unsqueeze(0)
    print("[config1] tri-att N=%d pad %d ending=%s" % (N, N - L, ending), flush=True)
    u = PF.tri_attn_block(z.to(DEV), W, mask.to(DEV), ending=ending, residual=False)
    torch.cuda.synchronize()
    ref = S.tri_attn(z.float(), P, mask, ending=ending, dtype=torch.float32)
    assert_bf16_close(u, ref, "config1 ending=%s" % ending)
    # dead attention rows: the uniform mean of v over all keys, gated and projected
    q, k, v, g, bias = S.triatt_prologue(z.float(), P, ending=ending, dtype=torch.float32)
    dead = torch.arange(L, N)
    o = v[:, dead].mean(dim=3, keepdim=True).expand(-1, -1, -1, N, -1).contiguous()          # [B, R, H, J, D]
    want = S.triatt_epilogue(o, g[:, dead], P, dtype=torch.float32)                          # [B, R, J, C] attention frame
    got = u[:, :, dead] if ending else u[:, dead]
    got = got.transpose(1, 2) if ending else got
    assert_bf16_close(got.cpu(), want, "config1 dead rows ending=%s" % ending)


# ------------------------------------------------------------------------------------------------------------------ metric shape
@pytest.mark.parametrize("ending", [False, True])
def test_metric_tri_attn_n768_sampled_rows_asymmetric_mask(ending):
    """The metric block's triangle attention (N = 768: the 8-wave block-layout core) on sampled attention rows against the
    statement restated per row, with an asymmetric mask (random keep pattern, a masked key band, a fully masked row) so a
    transposed or offset key mask would be caught."""
    from fpf_hip.attn import pair_fused as PF
    N = 768
    P = _ta_weights(21)
    W = _ta_pack(P)
    g = torch.Generator().manual_seed(22)
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16)
    mask = (torch.rand(1, N, N, generator=g) > 0.2).float()
    mask[:, :, 700:720] = 0
    mask[:, 5, :] = 0
    mask[:, :, 5] = 0
    rows = [0, 5, 127, 128, 255, 256, 383, 511, 640, 767]
    print("[metric] tri-att N=%d ending=%s" % (N, ending), flush=True)
    u = PF.tri_attn_block(z.to(DEV), W, mask.to(DEV), ending=ending, residual=False)
    torch.cuda.synchronize()
    u = u[0].cpu()
    got = u[:, rows].transpose(0, 1) if ending else u[rows]
    ref = S.tri_attn_rows(z[0].float(), P, mask[0], rows, ending=ending, dtype=torch.float32)
    assert_bf16_close(got, ref, "metric tri-att ending=%s rows %s" % (ending, rows))


@pytest.mark.parametrize("N", [800, 450, 97])
@pytest.mark.parametrize("ending", [False, True])
def test_tri_attn_any_n_sampled_rows(N, ending):
    """N not a multiple of 64: from N = 128 the block-layout core on a key axis padded to a multiple of 64 (the padding keys
    masked by the keep table, the padding queries never stored; N = 800 is the N <= 800 bucket's measured size), below it (97)
    the op core; with an asymmetric mask (a random keep pattern, a masked key band, a fully masked row) and no mask at all, on
    sampled attention rows against the statement restated per row; the whole output finite."""
    from fpf_hip.attn import pair_fused as PF
    P = _ta_weights(23)
    W = _ta_pack(P)
    g = torch.Generator().manual_seed(24)
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16)
    mask = (torch.rand(1, N, N, generator=g) > 0.2).float()
    mask[:, :, N - 40:N - 25] = 0
    mask[:, 7, :] = 0
    rows = sorted(set([0, 7, N // 3, N // 2, N - 65, N - 64, N - 2, N - 1]))
    for m in (mask, None):
        print("[any-N] tri-att N=%d ending=%s mask=%s" % (N, ending, m is not None), flush=True)
        u = PF.tri_attn_block(z.to(DEV), W, None if m is None else m.to(DEV), ending=ending, residual=False)
        torch.cuda.synchronize()
        assert torch.isfinite(u.float()).all()
        u = u[0].cpu()
        got = u[:, rows].transpose(0, 1) if ending else u[rows]
        ref = S.tri_attn_rows(z[0].float(), P, None if m is None else m[0], rows, ending=ending, dtype=torch.float32)
        assert_bf16_close(got, ref, "any-N tri-att N=%d ending=%s mask=%s rows %s" % (N, ending, m is not None, rows))


# ------------------------------------------------------------------------------------------------------------------ configs[3]
def test_config3_pairformer_layer_n512():
    """BASELINE configs[3]'s layer: N = 512, c_z = 128, c_s = 384, pair track bf16 (4 x 32 triangle heads), single track fp32
    (16 x 24 heads), s, z ~ N(0, 1), random-init weights, masks all ones; both outputs against the fp32 statements within the
    SAME_CLASS multiples of the stock layer with its pair stack under bf16 autocast."""
    from fpf_hip import pairformer as PFM
    N = 512
    params = _bf16_weights(PFM.random_params(seed=31))
    sp = PFM.random_single_params(c_s=384, heads=16, seed=32)
    for kk in ("w_q", "w_k", "w_v", "w_g", "w_o", "w_z"):
        sp["apb"][kk] = sp["apb"][kk].to(torch.bfloat16).float()
    g = torch.Generator().manual_seed(33)
    s = torch.randn(1, N, 384, generator=g)
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16)
    mask, pmask = torch.ones(1, N), torch.ones(1, N, N)
    blk, sb = PFM.PairBlock(params, DEV, torch.bfloat16), PFM.SingleBlock(sp, DEV)
    print("[config3] layer N=%d" % N, flush=True)
    zd = z.to(DEV)
    s_out, z_out = PFM.pairformer_layer(s.to(DEV), zd, mask.to(DEV), pmask.to(DEV), blk, sb)
    torch.cuda.synchronize()
    print("[config3] CPU statements", flush=True)
    s_ref, z_ref = S.pairformer_layer(s, z.float(), mask, pmask, dict(params, single=sp), dtype=torch.float32)
    z_ys = S.pair_block_autocast(z, pmask, params)
    s_ys = S.single_track(s, z_ys, mask, sp, dtype=torch.float32)
    assert_same_class(z_out.float(), z_ref, z_ys, "config3 layer z")
    assert_same_class(s_out, s_ref, s_ys, "config3 layer s")


# ------------------------------------------------------------------------------------------------------------------ block numerics
@pytest.mark.parametrize("N", [48, 96])
def test_pair_block_same_class(N):
    """The bf16 pair block with padded residues against the fp32 statements: within the SAME_CLASS multiples of the bf16-autocast
    statement (the class the reference admits a bf16 block in; the per-op absolute bars are held by each op's tests)."""
    from fpf_hip import pairformer as PFM
    params = _bf16_weights(PFM.random_params(seed=N))
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(N + 1)).to(torch.bfloat16)
    mask = torch.ones(1, N, N)
    mask[:, N - 4:, :] = 0
    mask[:, :, N - 4:] = 0
    blk = PFM.PairBlock(params, DEV, torch.bfloat16)
    zd = z.to(DEV)
    PFM.pair_block(zd, mask.to(DEV), blk)
    torch.cuda.synchronize()
    ref = S.pair_block(z.float(), mask, params, dtype=torch.float32)
    assert_same_class(zd.float(), ref, S.pair_block_autocast(z, mask, params), "pair block N=%d" % N)


@pytest.mark.parametrize("N", [96, 160])
def test_pair_block_batch2_same_class_and_entries_independent(N):
    """Two batch entries with different masks (entry 0 padded by 6 residues on both axes, entry 1 a random pair mask with two
    dead rows): the B = 2 pair block against the fp32 statements at SAME_CLASS, and each entry bitwise equal to a B = 1 block
    on that entry alone (no kernel mixes entries, whatever the grid).  N = 96 runs the generic tri-att core, N = 160 the
    block-layout core with its key axis padded to 192."""
    from fpf_hip import pairformer as PFM
    params = _bf16_weights(PFM.random_params(seed=N + 3))
    g = torch.Generator().manual_seed(N + 5)
    z = torch.randn(2, N, N, 128, generator=g).to(torch.bfloat16)
    mask = torch.ones(2, N, N)
    mask[0, N - 6:, :] = 0
    mask[0, :, N - 6:] = 0
    mask[1] = (torch.rand(N, N, generator=g) > 0.15).float()
    mask[1, 7:9, :] = 0
    blk = PFM.PairBlock(params, DEV, torch.bfloat16)
    print("[case] pair block B=2 N=%d" % N, flush=True)
    zd, md = z.to(DEV), mask.to(DEV)
    PFM.pair_block(zd, md, blk)
    singles = []
    for e in range(2):
        ze = z[e:e + 1].to(DEV)
        PFM.pair_block(ze, md[e:e + 1].contiguous(), blk)
        singles.append(ze)
    torch.cuda.synchronize()
    assert torch.isfinite(zd.float()).all()
    for e in range(2):
        assert torch.equal(zd[e:e + 1], singles[e]), "entry %d of the batch differs from the block on it alone" % e
    ref = S.pair_block(z.float(), mask, params, dtype=torch.float32)
    assert_same_class(zd.float(), ref, S.pair_block_autocast(z, mask, params), "pair block B=2 N=%d" % N)


def test_pair_block_per_site_budget():
    """Where the block's error comes from, on the smoke's inputs (N = 48, 4 padded residues, seed-1 weights): each site alone,
    fed the same bf16 input (the fp32 chain's state rounded to bf16), its update against the fp32 statement of that site, next
    to the bf16-autocast statement's update on the same input -- each held to SAME_CLASS -- and the share of the block error
    that the bf16 residual stream alone causes (the fp32 chain with z rounded to bf16 after every site: the resident-z
    composition rounds there, the autocast statement keeps z in fp32)."""
    from fpf_hip import pairformer as PFM
    from fpf_hip.attn import pair_fused as PF
    from fpf_hip.kernels import transition as TR
    from fpf_hip.kernels import trimul as TM
    N = 48
    params = _bf16_weights(PFM.random_params(seed=1))
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).float()
    mask = torch.ones(1, N, N)
    mask[:, N - 4:, :] = 0
    mask[:, :, N - 4:] = 0
    blk = PFM.PairBlock(params, DEV, torch.bfloat16)
    t = params["tr"]
    sites = [
        ("trimul_out", lambda x: S.trimul(x, mask, direction="outgoing", weights=params["tmo"], dtype=torch.float32),
         lambda x: S.trimul_autocast(x, mask, direction="outgoing", weights=params["tmo"]),
         lambda xd: TM.triangle_multiplication(xd, mask.to(DEV), direction="outgoing", weights=blk.tmo, word="fast", cache=blk.cache_o)),
        ("trimul_in", lambda x: S.trimul(x, mask, direction="incoming", weights=params["tmi"], dtype=torch.float32),
         lambda x: S.trimul_autocast(x, mask, direction="incoming", weights=params["tmi"]),
         lambda xd: TM.triangle_multiplication(xd, mask.to(DEV), direction="incoming", weights=blk.tmi, word="fast", cache=blk.cache_i)),
        ("tri_att_start", lambda x: S.tri_attn(x, params["tas"], mask, ending=False, dtype=torch.float32),
         lambda x: S.tri_attn_autocast(x, params["tas"], mask, ending=False),
         lambda xd: PF.tri_attn_block(xd, blk.ta["tas"], mask.to(DEV), ending=False)),
        ("tri_att_end", lambda x: S.tri_attn(x, params["tae"], mask, ending=True, dtype=torch.float32),
         lambda x: S.tri_attn_autocast(x, params["tae"], mask, ending=True),
         lambda xd: PF.tri_attn_block(xd, blk.ta["tae"], mask.to(DEV), ending=True)),
        ("transition", lambda x: S.transition(x, t["w_a"], t["w_b"], t["w_o"], t["ln_w"], t["ln_b"], dtype=torch.float32),
         lambda x: S.transition_autocast(x, t["w_a"], t["w_b"], t["w_o"], t["ln_w"], t["ln_b"]),
         lambda xd: TR.transition(xd, blk.tr, word="fast")[0]),
    ]
    x32 = z.clone()          # the fp32 chain
    xr = z.clone()           # the fp32 chain with the residual stream rounded to bf16 after every site
    for name, f32, ac, hip in sites:
        xin = x32.to(torch.bfloat16).float()                           # the site's input, bf16-representable
        ref = f32(xin)
        u = hip(xin.to(torch.bfloat16).to(DEV))
        torch.cuda.synchronize()
        assert_same_class(u.float().cpu(), ref, ac(xin), "site %s" % name)
        x32 = x32 + f32(x32)
        xr = (xr + f32(xr)).to(torch.bfloat16).float()
    ma, rl = max_abs(xr, x32), rel_l2(xr, x32)
    print("[same-class] block: the bf16 residual stream alone (exact sites) max_abs=%.3e rel_l2=%.3e vs the fp32 chain" % (ma, rl))


# ------------------------------------------------------------------------------------------------------------------ biases
@pytest.mark.parametrize("ending", [False, True])
def test_block_gate_and_output_biases(ending):
    """b_g (gate projection bias) and b_o (output projection bias), as the openfold3 kits pass them
    (openfold3_opt/cells/pairfused.py:396-399): the fused bf16 block and the fp32 block against the statement with the biases,
    and the staged bf16 path (prologue adds b_g to g, epilogue adds b_o) against the same."""
    from fpf_hip.attn import pair_fused as PF
    N = 96
    P = _ta_weights(41, biases=True)
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(42)).to(torch.bfloat16)
    mask = torch.ones(1, N, N)
    mask[:, :, N - 6:] = 0
    zd, md = z.to(DEV), mask.to(DEV)
    W = _ta_pack(P)
    print("[bias] bf16 block ending=%s" % ending, flush=True)
    u = PF.tri_attn_block(zd, W, md, ending=ending, residual=False)
    torch.cuda.synchronize()
    ref = S.tri_attn(z.float(), P, mask, ending=ending, dtype=torch.float32)
    assert_bf16_close(u, ref, "bf16 block with b_g, b_o ending=%s" % ending)
    nob = S.tri_attn(z.float(), {k: v for k, v in P.items() if k not in ("b_g", "b_o")}, mask, ending=ending, dtype=torch.float32)
    assert max_abs(ref, nob) > 0.1                                  # the biases change the result on these inputs
    print("[bias] staged bf16 ending=%s" % ending, flush=True)
    q, k, v, g, bias = PF.prologue(zd, W, ending=ending)
    o = PF.core_attention(q, k, v, bias, PF._key_mask(md, zd, ending))
    us = PF.epilogue(o, g, W, ending=ending, residual=False)
    torch.cuda.synchronize()
    assert_bf16_close(us.transpose(1, 2) if ending else us, ref, "staged bf16 with b_g, b_o ending=%s" % ending)
    print("[bias] fp32 block ending=%s" % ending, flush=True)
    Wf = _ta_pack(P, torch.float32)
    uf = PF.tri_attn_block(z.float().to(DEV), Wf, md, ending=ending, residual=False, word="exact")
    torch.cuda.synchronize()
    ref64 = S.tri_attn(z.double(), P, mask, ending=ending, dtype=torch.float64)
    live = slice(0, N - 6)
    assert_f32_close(uf[:, :, live] if ending else uf, ref64[:, :, live] if ending else ref64, "fp32 block with b_g, b_o ending=%s" % ending)


# ------------------------------------------------------------------------------------------------------------------ run contract
def test_masked_block_under_inference_mode():
    """boltz predicts under torch.inference_mode(): a mask created there is an inference tensor (no version counter).  The block
    serves it (converting it on every call) and equals the same call outside inference mode bit for bit."""
    from fpf_hip.attn import pair_fused as PF
    N = 128
    P = _ta_weights(51)
    W = _ta_pack(P)
    z = torch.randn(1, N, N, 128, generator=torch.Generator().manual_seed(52)).to(torch.bfloat16).to(DEV)
    m0 = torch.ones(1, N, N)
    m0[:, :, N - 9:] = 0
    want = PF.tri_attn_block(z, W, m0.to(DEV), ending=True, residual=False)
    with torch.inference_mode():
        mi = m0.to(DEV)
        assert mi.is_inference()
        got = PF.tri_attn_block(z, W, mi, ending=True, residual=False)
        got2 = PF.tri_attn_block(z, W, mi, ending=True, residual=False)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(got2, want)


def _layer_setup(N, seed):
    from fpf_hip import pairformer as PFM
    params = PFM.random_params(seed=seed)
    sp = PFM.random_single_params(c_s=384, heads=16, seed=seed + 1)
    g = torch.Generator().manual_seed(seed + 2)
    z = (torch.randn(1, N, N, 128, generator=g) * 2.0).to(torch.bfloat16).to(DEV)
    s = torch.randn(1, N, 384, generator=g).to(DEV)
    mask = torch.ones(1, N, device=DEV)
    mask[:, N - 7:] = 0
    pmask = mask[:, :, None] * mask[:, None, :]
    return PFM.PairBlock(params, DEV, torch.bfloat16), PFM.SingleBlock(sp, DEV), z, s, mask, pmask


@pytest.mark.parametrize("N", [384, 397])
def test_layer_repeated_runs_bitwise(N):
    """The whole layer (five in-place pair sites, then the single track) is bitwise identical over 20 repetitions, at a size the
    tiles divide and at one they do not (397): no race in the in-place stores and no order-dependent reduction (fixed tiles,
    no atomics, no split-K)."""
    from fpf_hip import pairformer as PFM
    blk, sb, z, s, mask, pmask = _layer_setup(N, 61)
    print("[repeat] layer N=%d x 20" % N, flush=True)
    outs = []
    for _ in range(20):
        zr = z.clone()
        s_out, _ = PFM.pairformer_layer(s, zr, mask, pmask, blk, sb)
        outs.append((zr, s_out))
    torch.cuda.synchronize()
    assert not torch.equal(outs[0][0], z)
    for rep in range(1, 20):
        assert torch.equal(outs[rep][0], outs[0][0]) and torch.equal(outs[rep][1], outs[0][1]), "run %d differs from run 0" % rep


def test_layer_no_host_sync_after_first_call():
    """After one eager call with a given mask tensor, a second call of the whole layer issues no synchronising operation
    (torch.cuda.set_sync_debug_mode('error') raises on any): weight packs, masks, scratch and device facts are cached, and
    the library never synchronises.  The same holds under inference_mode, whose mask tensors are converted per call."""
    from fpf_hip import pairformer as PFM
    blk, sb, z, s, mask, pmask = _layer_setup(160, 71)
    for inference in (False, True):
        ctx = torch.inference_mode() if inference else torch.no_grad()
        with ctx:
            zz, pm = z.clone(), pmask.clone()
            PFM.pairformer_layer(s, zz, mask, pm, blk, sb)                       # first call: eager set-up
            torch.cuda.synchronize()
            torch.cuda.set_sync_debug_mode("error")
            try:
                PFM.pairformer_layer(s, zz, mask, pm, blk, sb)
            finally:
                torch.cuda.set_sync_debug_mode("default")
        torch.cuda.synchronize()


@pytest.mark.parametrize("N,masked", [(200, True), (768, False)])
def test_pair_block_graph_replays_equal_eager(N, masked):
    """The pair block captured into a HIP graph (torch.cuda.graph on a side stream, after one eager call there sized that
    stream's shared scratch) replays the eager block's bits: three replays from the same z, with eager work and a
    synchronisation between them, each bitwise equal to the eager block on the same input and finite -- the library records
    no memset nodes and keeps no host-side state that a replay would skip.  N = 200 with a random mask, dead rows and masked
    trailing keys runs the keep table, the masked core and its fallback check; N = 768 without a mask the metric's path."""
    from fpf_hip import pairformer as PFM
    g = torch.Generator().manual_seed(N + 17)
    blk = PFM.PairBlock(PFM.random_params(seed=7), DEV, torch.bfloat16)
    z0 = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16).to(DEV)
    m = torch.ones(1, N, N)
    if masked:
        m = (torch.rand(1, N, N, generator=g) > 0.2).float()
        m[:, 3:7, :] = 0                                  # dead rows
        m[:, :, N - 9:] = 0                               # trailing keys masked in every row
    mask = m.to(DEV)
    print("[case] graph replay N=%d masked=%s" % (N, masked), flush=True)
    eager, ze = [], z0.clone()
    for _ in range(3):
        PFM.pair_block(ze, mask, blk)
        eager.append(ze.clone())
    torch.cuda.synchronize()
    zg = z0.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        PFM.pair_block(zg, mask, blk)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        PFM.pair_block(zg, mask, blk)
    torch.cuda.synchronize()
    zg.copy_(z0)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(zg.float()).all(), "replay %d: non-finite" % i
        assert torch.equal(zg, eager[i]), "replay %d differs from the eager block" % i
        PFM.pair_block(z0.clone(), mask, blk)             # eager work between replays
        torch.cuda.synchronize()
    del graph
    torch.cuda.synchronize()

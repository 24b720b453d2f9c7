"""Host logic of the provider faces (no GPU): row / tier-word selection, refusals by name before any launch, the weight
vocabulary, and the one-GPU guard of bench.py."""
import os
import subprocess
import sys

import pytest
import torch

from conftest import ROOT


def test_tier_words_map_to_rows_by_dtype():
    from fpf_hip import _face as F
    assert F.resolve("fast", "bf16", "gfx950", "t").row == F.ROW_FAST
    assert F.resolve("big", "bf16", "gfx950", "t").row == F.ROW_FAST
    assert F.resolve("fast", "fp32", "gfx950", "t").row == F.ROW_F32
    assert F.resolve("exact", "fp32", "gfx950", "t").row == F.ROW_F32
    assert F.resolve("hip_gfx950", "bf16", "gfx950", "t").cls == "fast"
    assert F.resolve("hip_gfx950_f32", "fp32", "gfx950", "t").cls == "exact"


@pytest.mark.parametrize("word,dt,arch,kind,fallback", [
    ("exact", "bf16", "gfx950", "exact:bf16_input", "stock"),
    ("fast", "bf16", "gfx942", "arch:gfx942", "stock"),
    ("fast", "bf16", "cpu", "arch:cpu", "stock"),
    ("hip_gfx950", "fp32", "gfx950", "dtype:fp32", "hip_gfx950_f32"),
    ("hip_gfx950_f32", "bf16", "gfx950", "dtype:bf16", "hip_gfx950"),
    ("flash", "bf16", "gfx950", "unknown_word:flash", "stock"),
    ("fast", "fp16", "gfx950", "dtype:fp16", "hip_gfx950"),
])
def test_refusals_name_kind_and_fallback(word, dt, arch, kind, fallback):
    from fpf_hip import _face as F
    with pytest.raises(F.Refusal) as e:
        F.resolve(word, dt, arch, "t")
    assert e.value.kind == kind and e.value.fallback == fallback
    with pytest.raises(F.Refusal) as e2:                # the memo re-raises the same refusal
        F.resolve(word, dt, arch, "t")
    assert e2.value.kind == kind


def test_stock_row_is_the_callers_own_and_word_is_required():
    from fpf_hip import _face as F
    with pytest.raises(F.Refusal) as e:
        F.resolve("stock", "bf16", "gfx950", "t")
    assert e.value.fallback is None
    with pytest.raises(ValueError):
        F.resolve(None, "bf16", "gfx950", "t")


def test_triattn_select_head_dim_rows():
    from fpf_hip.kernels import triattn as TA
    assert TA.select("gfx950", torch.bfloat16, 32, 4, 768, word="fast").row == "hip_gfx950"
    with pytest.raises(TA.Refusal) as e:
        TA.select("gfx950", torch.bfloat16, 16, 4, 512, word="fast")
    assert e.value.kind == "no_row:head_dim16" and e.value.fallback == "hip_gfx950_f32"
    assert TA.select("gfx950", torch.float32, 16, 4, 512, word="exact").row == "hip_gfx950_f32"
    with pytest.raises(TA.Refusal):
        TA.select("gfx950", torch.float32, 24, 16, 512, word="exact")
    with pytest.raises(TA.Refusal) as e:
        TA.select("gfx950", torch.bfloat16, 32, 4, 768, direction="bwd", word="fast")
    assert e.value.kind.startswith("direction")


def test_trimul_select_and_weight_vocabulary():
    from fpf_hip.kernels import trimul as TM
    assert set(TM.WEIGHT_KEYS) == {"ln_in_w", "ln_in_b", "w_ag", "w_ap", "w_bg", "w_bp", "ln_out_w", "ln_out_b", "w_o", "w_og"}
    assert len(TM.WEIGHT_KEYS) == 10
    assert TM.select("gfx950", torch.bfloat16, 128, 128, 768, "outgoing", word="fast").row == "hip_gfx950"
    assert TM.select("gfx950", torch.float32, 64, 32, 100, "incoming", word="exact").row == "hip_gfx950_f32"


def test_ln_select_cols_gate():
    from fpf_hip.kernels import ln as LN
    assert LN.select((9, 5), torch.bfloat16, None, 768, word="fast", C=128).row == "hip_gfx950"
    with pytest.raises(LN.Refusal):
        LN.select("9.5", torch.bfloat16, None, 768, word="fast", C=2048)
    with pytest.raises(LN.Refusal) as e:
        LN.select("9.5", "bf16", None, 768, word="fast", C=128, pass_="bwd")
    assert e.value.kind == "no_backward"


def test_cpu_tensors_are_refused_by_name_before_any_launch():
    """A host tensor resolves to the 'cpu' device word and is refused; nothing reaches the library."""
    from fpf_hip.kernels import ln as LN
    from fpf_hip.kernels import triattn as TA
    x = torch.randn(4, 128)
    with pytest.raises(LN.Refusal) as e:
        LN.layer_norm(x, (128,), None, None, 1e-5, word="fast")
    assert e.value.kind == "arch:cpu"
    q = torch.randn(1, 2, 4, 8, 32, dtype=torch.bfloat16)
    with pytest.raises(TA.Refusal):
        TA.triangle_attention(q, q, q, torch.zeros(1, 1, 4, 8, 8), None, word="fast")


def test_pair_fused_refuses_unsupported_packs():
    from fpf_hip.attn import pair_fused as PF
    w = torch.randn(128, 128)
    Wb = PF.pack_triattn_weights(w_o=w, n_heads=4, head_dim=32, w_q=w, w_k=w, w_v=w, w_g=w, w_b=torch.randn(4, 128), b_o=torch.zeros(128),
                                 b_g=torch.ones(128))
    assert Wb.b_o is not None and Wb.b_g is not None
    with pytest.raises(PF.Unsupported) as e:
        PF.pack_triattn_weights(w_o=w, n_heads=4, head_dim=32, w_q=w, w_k=w, w_v=w, w_g=w, w_b=torch.randn(4, 128), b_g=torch.ones(129))
    assert e.value.reason == "b_g-shape"
    with pytest.raises(PF.Unsupported) as e:
        PF.pack_triattn_weights(w_o=w, n_heads=4, head_dim=32, w_q=w, w_k=w, w_v=w, w_g=w, w_b=torch.randn(4, 128), b_o=torch.zeros(64))
    assert e.value.reason == "b_o-shape"
    with pytest.raises(PF.Unsupported) as e:
        PF.pack_triattn_weights(w_o=w, n_heads=4, head_dim=32, w_q=w, w_k=w, w_v=w, w_g=None, w_b=torch.randn(4, 128))
    assert e.value.reason == "gate:none"
    W = PF.pack_triattn_weights(w_o=w, n_heads=4, head_dim=32, w_q=w, w_k=w, w_v=w, w_g=w, w_b=torch.randn(4, 128))
    with pytest.raises(PF.Unsupported) as e:           # host z: refused by the row gate, before the library
        PF.tri_attn_block(torch.randn(1, 8, 8, 128), W, ending=False)
    assert e.value.reason == "arch:cpu"
    km = PF._key_mask(torch.tensor([[[1.0, 0.0], [1.0, 1.0]]]), None, ending=True)
    assert km.shape == (1, 2, 1, 1, 2) and km[0, 0, 0, 0].tolist() == [True, True] and km[0, 1, 0, 0].tolist() == [False, True]


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2, r.stderr
    assert "single MI355X" in r.stderr


def test_cell_keys_follow_the_reference_grammar_and_bucket_rule():
    from fpf_hip import cells as C
    assert C.bucket(1) == (256, True) and C.bucket(511) == (511, True) and C.bucket(512) == (800, True)
    assert C.bucket(2049) == (2048, False)                     # above the largest listed size: its cell, unmeasured
    assert C.triattn_key("bf16", 32, 4, 768) == "9.5|bf16|D32|H4|N<=800|fwd"
    assert C.trimul_key("bf16", 128, 128, 384, "in") == "9.5|bf16|C128|H128|N<=400|in|fwd"
    assert C.transition_key("fp32", 128, 4, 300) == "9.5|fp32|pair_c128_n4|N<=400|eager|fwd"
    from fpf_hip.kernels import triattn as TA
    from fpf_hip.kernels import trimul as TM
    assert TA.select("gfx950", torch.bfloat16, 32, 4, 768, word="fast").cell == "9.5|bf16|D32|H4|N<=800|fwd"
    assert TM.select("gfx950", torch.bfloat16, 128, 128, 768, "outgoing", word="fast").cell == "9.5|bf16|C128|H128|N<=800|out|fwd"


def test_measured_table_covers_every_bucket_and_follows_the_exact_rule():
    """The committed MI355X column: every (face, dtype, bucket[, direction]) cell measured; 'fast' is the bf16 row; 'exact'
    is the fp32 row exactly where it measured at least as fast as the fp32 torch statement (the reference's exact rule)."""
    from fpf_hip import cells as C
    t = C.table()
    assert set(("triattn", "trimul", "transition")) <= set(t)
    for n in C.BUCKETS:
        for dw in ("bf16", "fp32"):
            keys = {"triattn": [C.triattn_key(dw, 32, 4, n)], "transition": [C.transition_key(dw, 128, 4, n)],
                    "trimul": [C.trimul_key(dw, 128, 128, n, d) for d in ("in", "out")]}
            for face, ks in keys.items():
                for k in ks:
                    c = C.lookup(face, k)
                    assert c is not None, k
                    row = "hip_gfx950" if dw == "bf16" else "hip_gfx950_f32"
                    assert c["ms"][row] > 0 and c["stock_ms"] > 0
                    if dw == "bf16":
                        assert c["fast"] == row
                    else:
                        assert c["exact"] == (row if c["stock_ms"] >= c["ms"][row] else "stock"), k


def test_exact_word_follows_the_measured_cell():
    from fpf_hip import cells as C
    from fpf_hip.kernels import trimul as TM
    from fpf_hip.kernels import triattn as TA
    for n in (100, 768, 2000):
        cell = C.lookup("trimul", C.trimul_key("fp32", 128, 128, n, "out"))
        if cell["exact"] == "stock":
            with pytest.raises(TM.Refusal) as e:
                TM.select("gfx950", torch.float32, 128, 128, n, "outgoing", word="exact")
            assert e.value.kind == "exact:stock_faster" and e.value.fallback == "stock"
        else:
            assert TM.select("gfx950", torch.float32, 128, 128, n, "outgoing", word="exact").row == "hip_gfx950_f32"
        # the row name always serves the row
        assert TM.select("gfx950", torch.float32, 128, 128, n, "outgoing", word="hip_gfx950_f32").row == "hip_gfx950_f32"
        cell = C.lookup("triattn", C.triattn_key("fp32", 32, 4, n))
        assert (TA.select("gfx950", torch.float32, 32, 4, n, word="exact").row == "hip_gfx950_f32") == (cell["exact"] == "hip_gfx950_f32")


# ------------------------------------------------------------------------------------------------------------- drop-in contract
@pytest.mark.parametrize("cc", [(9, 5), [9, 5], "9.5", 9.5, "sm_95", "gfx950", "gfx950:sramecc+:xnack-"])
def test_capability_forms_name_the_mi355x(cc):
    from fpf_hip import _face as F
    assert F.arch_word(cc) == "gfx950"


def test_kit_trimul_probe_resolves_a_hip_selection():
    """The boltz2 kit's probe (boltz2/opt/boltz2_opt/trimul.py:160-166): select(cc, "bf16", 128, 128, 512, d, word=..., stack=...)
    then admits(sel.row, cc, "bf16", 128, 128, 512, backward=False, residual=False, batch=1, abi=None), with the capability ROCm
    torch reports for an MI355X."""
    from fpf_hip.kernels import trimul as KT
    cc = (9, 5)
    for d in ("outgoing", "incoming"):
        sel = KT.select(cc, "bf16", 128, 128, 512, d, word="fast", stack=None)
        assert sel.row == "hip_gfx950"
        assert KT.admits(sel.row, cc, "bf16", 128, 128, 512, backward=False, residual=False, batch=1, abi=None) is None
    with pytest.raises(KT.Refusal) as e:
        KT.select((9, 0), "bf16", 128, 128, 512, "outgoing", word="fast")
    assert e.value.kind == "arch:cc9.0"
    with pytest.raises(KT.Refusal) as e:
        KT.admits("hip_gfx950", cc, "bf16", 128, 128, 512, backward=True)
    assert e.value.kind == "no_backward"
    with pytest.raises(KT.Refusal) as e:
        KT.select(cc, "bf16", 128, 128, 512, "outgoing", word="fast", exclude=("hip_gfx950",))
    assert e.value.kind == "excluded:hip_gfx950"
    assert KT.precision_word("bf16", "fp32") == "f32z_bf16" and KT.precision_word(torch.float32, tf32=True) == "tf32"
    assert KT.select(cc, torch.float32, 128, 128, 100, "outgoing", word="hip_gfx950_f32", tf32=True).row == "hip_gfx950_f32"


def test_select_keywords_are_served_or_refused_by_name():
    from fpf_hip.kernels import triattn as TA
    from fpf_hip.kernels import trimul as TM
    assert TA.select("9.5", "bf16", 32, 4, 768, word="fast", prefer=("hip_gfx950",), stack="rocm7", form=None, lib=None).row == "hip_gfx950"
    with pytest.raises(TA.Refusal) as e:                       # prefer narrows a tier word to rows this package does not have
        TA.select("9.5", "bf16", 32, 4, 768, word="fast", prefer=("cuda_sm90a", "k2b"))
    assert e.value.kind == "prefer_excludes:hip_gfx950"
    with pytest.raises(TA.Refusal) as e:                       # a launch setting is refused, never ignored
        TA.select((9, 5), "bf16", 32, 4, 768, word="fast", config={"BLOCK_M": 64})
    assert e.value.kind == "config:fixed_launch"
    with pytest.raises(TA.Refusal) as e:
        TA.select((9, 5), "bf16", 32, 4, 768, word="hip_gfx950@bm64")
    assert e.value.kind == "config_word:bm64"
    assert TA.admits("hip_gfx950", (9, 5), "bf16", 32, 4, 768) == (True, "ok")
    assert TA.admits("hip_gfx950", (9, 5), "bf16", 16, 4, 768) == (False, "no_row:head_dim16")
    assert TA.admits("cuda_sm90a", (9, 5), "bf16", 32, 4, 768)[0] is False
    # the f32z_bf16 class (an fp32 pair tensor under bf16 autocast) is served by the bf16 row (fp32 z / out, bf16 operands)
    assert TM.select((9, 5), "bf16", 128, 128, 400, "outgoing", word="fast", residency="fp32").row == "hip_gfx950"
    assert TM.admits("hip_gfx950", (9, 5), "bf16", 128, 128, 400, residency="fp32") is None
    assert TM.call_precision(torch.zeros(2, 2, 2, 128))[0] == "fp32"
    assert TM.call_precision(torch.zeros(2, 2, 2, 128, dtype=torch.bfloat16)) == ("bf16", torch.bfloat16)


def test_kit_transition_select_and_ln_given():
    """boltz2/opt/boltz2_opt/transition.py:149: select(word, c=, hidden=, n_tokens=, dtype="bf16", family=, residual=, mask=, cc=,
    stack=, rows_count=, ln_given=); the caller's own LayerNorm output (ln_given) is served by the bf16 row and refused by name on
    the fp32 row."""
    from fpf_hip.kernels import transition as KT
    sel = KT.select("fast", c=128, hidden=512, n_tokens=768, dtype="bf16", family="pair", residual=False, mask=False, cc=(9, 5), stack=None,
                    rows_count=768 * 768, ln_given=False)
    assert sel.row == "hip_gfx950"
    assert KT.select("fast", c=128, hidden=512, n_tokens=768, dtype="bf16", cc=(9, 5), ln_given=True).row == "hip_gfx950"
    with pytest.raises(KT.Refusal) as e:
        KT.select("exact", c=128, hidden=512, n_tokens=768, dtype="fp32", cc=(9, 5), ln_given=True)
    assert e.value.kind == "ln_given"
    with pytest.raises(KT.Refusal) as e:
        KT.select("fast", c=128, hidden=512, dtype="bf16", cc=(9, 5), form="geglu")
    assert e.value.kind == "form:geglu"


def _pack_small():
    from fpf_hip.attn import pair_fused as PF
    w = torch.randn(128, 128)
    return PF.pack_triattn_weights(w_o=w, n_heads=4, head_dim=32, w_q=w, w_k=w, w_v=w, w_g=w, w_b=torch.randn(4, 128))


@pytest.mark.parametrize("kw,reason", [
    (dict(ln="stock"), "ln:stock-needs-x_ln"),
    (dict(x_ln=torch.zeros(1, 8, 8, 128)), "x_ln:ln_fused"),
    (dict(ln="layer"), "ln:layer"),
    (dict(impl="torch"), "impl:torch"),
    (dict(core="flash_triattn"), "core:flash_triattn"),
    (dict(core="k2b"), "core:k2b"),
    (dict(bias_frame="q"), "bias_frame:q"),
    (dict(variant="v3"), "variant:v3"),
])
def test_block_keywords_not_served_are_refused_by_name(kw, reason):
    """Nothing is swallowed: an exact-construction or foreign-core call is refused before any launch (these run on host
    tensors, so a call that got past the keyword gate would be refused 'arch:cpu' instead)."""
    from fpf_hip.attn import pair_fused as PF
    W = _pack_small()
    with pytest.raises(PF.Unsupported) as e:
        PF.tri_attn_block(torch.randn(1, 8, 8, 128), W, **kw)
    assert e.value.reason == reason
    T = PF.pack_transition_weights(w_out=torch.randn(128, 512), w_a=torch.randn(512, 128), w_b=torch.randn(512, 128))
    with pytest.raises(PF.Unsupported) as e:
        PF.transition(torch.randn(1, 8, 8, 128), T, ln="stock")
    assert e.value.reason == "ln:stock-needs-x_ln"
    with pytest.raises(PF.Unsupported) as e:                  # x_ln must be bf16 of x's shape
        PF.transition(torch.randn(1, 8, 8, 128), T, ln="stock", x_ln=torch.randn(1, 8, 8, 128))
    assert e.value.reason == "x_ln-shape"
    with pytest.raises(PF.Unsupported) as e:
        PF.transition(torch.randn(1, 8, 8, 128), T, variant="v1")
    assert e.value.reason == "variant:v1"
    with pytest.raises(PF.Unsupported) as e:
        PF.prologue(torch.randn(1, 8, 8, 128), W, write_x=True)
    assert e.value.reason == "write_x"


def test_core_attention_hands_a_callable_core_a_unit_stride_v():
    from fpf_hip.attn import pair_fused as PF
    q = torch.randn(1, 2, 4, 8, 32)
    vs = torch.randn(1, 2, 4, 32, 8)
    v = vs.transpose(-1, -2)                                   # the prologue's transposed V^T view
    seen = {}

    def core(q_, k_, v_, b_, m_, sc):
        seen["stride"] = v_.stride(-1)
        seen["equal"] = torch.equal(v_, v)
        return q_
    PF.core_attention(q, q, v, torch.zeros(1, 1, 4, 8, 8), None, core=core)
    assert seen == {"stride": 1, "equal": True}


def test_pair_mask_under_inference_mode_and_on_another_device():
    """A mask made under torch.inference_mode() has no version counter: converted on every call, never cached; a mask on another
    device is moved to z's device before any launch (a meta z stands in for the GPU here)."""
    from fpf_hip.attn import pair_fused as PF
    z4 = torch.zeros(1, 6, 6, 128)
    with torch.inference_mode():
        m = torch.ones(1, 6, 6)
        m[:, :, 4:] = 0
        u8, dt, frame = PF._pair_mask(m, z4, ending=True)
        u8b, _, _ = PF._pair_mask(m, z4, ending=True)
    assert frame == 1 and u8.dtype == torch.uint8 and u8[0, 0].tolist() == [1, 1, 1, 1, 1, 1] and u8[0, 5].tolist() == [0] * 6
    assert torch.equal(u8, u8b)
    zm = torch.empty(1, 6, 6, 128, device="meta")
    u8m, _, _ = PF._pair_mask(torch.ones(1, 6, 6), zm)
    assert u8m.device.type == "meta"
    km = PF._key_mask(torch.ones(1, 6, 6), zm, ending=False)
    assert km.device.type == "meta"


def test_shared_scratch_is_one_buffer_per_stream_sized_by_the_largest_call():
    """The trunk holds ONE workspace for all its layers and sites: the largest of the per-call needs, not their sum."""
    from fpf_hip import _face as F
    from fpf_hip import _lib as L
    F.release_scratch()
    a = F.scratch("cpu", 100)
    b = F.scratch("cpu", 50)
    assert a.data_ptr() == b.data_ptr() and F.scratch_bytes("cpu") == 100
    c = F.scratch("cpu", 300)
    assert c.numel() == 300 and F.scratch_bytes("cpu") == 300
    F.scratch("cpu", 10, kind="bias")
    assert F.scratch_bytes("cpu") == 310
    F.release_scratch()
    lib = L.lib()
    for N, cap in ((512, 3e9), (768, 3e9)):                  # 48 layers x (2 trimul + 2 tri-att): one buffer of the largest need
        need = max(lib.fpf_trimul_workspace_bytes(1, N, 128, 128, L.DT_BF16), lib.fpf_triattn_block_workspace_bytes(1, N, 0, 128, 4, 32, L.DT_BF16))
        assert need < cap, (N, need)


def test_shared_scratch_keeps_an_outgrown_buffer_a_captured_call_used():
    """A buffer handed out under graph capture is marked; when a larger call outgrows it, it stays allocated (a graph replays with
    its address), while unmarked buffers go back to the allocator; release_scratch drops both."""
    from fpf_hip import _face as F
    F.release_scratch()
    t = F.scratch("cpu", 100)
    t._fpf_captured = True                       # what a call under capture leaves on the buffer it was handed
    t2 = F.scratch("cpu", 300)
    assert t2.numel() >= 300 and t2.data_ptr() != t.data_ptr()
    assert any(c is t for c in F._CAPTURED)
    F.scratch("cpu", 600)                        # t2 was never captured: not kept
    assert not any(c is t2 for c in F._CAPTURED)
    assert F.reserve_scratch("cpu", 50).numel() >= 600
    F.release_scratch()
    assert F._CAPTURED == [] and F.scratch_bytes() == 0


def test_block_mask_all_ones_is_handed_on_as_no_mask():
    """The block face converts a pair mask once per tensor (object and version); one that keeps every pixel is handed on as no
    mask (bz_pairfuse.py:46-50: a trivial mask goes to the providers as None), in both frames; a mask with a masked pixel, a
    mask changed in place and an inference-mode mask (converted per call) are handed on as u8."""
    from fpf_hip import _lib as L
    from fpf_hip.attn import pair_fused as PF
    z4 = torch.zeros(1, 8, 8, 128, dtype=torch.bfloat16)
    ones = torch.ones(1, 8, 8)
    for ending in (False, True):
        for _ in range(2):                                           # the conversion and the cached answer
            assert PF._pair_mask(ones, z4, ending) == (None, L.DT_U8, 0)
    part = torch.ones(1, 8, 8)
    part[0, 3, 5] = 0
    m, dt, frame = PF._pair_mask(part, z4, True)
    assert frame == 1 and dt == L.DT_U8 and m.dtype == torch.uint8 and int(m[0, 5, 3]) == 0 and int(m.sum()) == 63
    ones[0, 1, 2] = 0                                                # in place: a new version, converted again
    m, _, frame = PF._pair_mask(ones, z4, False)
    assert frame == 1 and int(m[0, 1, 2]) == 0
    with torch.inference_mode():
        inf = torch.ones(1, 8, 8)
        m, _, frame = PF._pair_mask(inf, z4, False)
    assert frame == 1 and int(m.sum()) == 64

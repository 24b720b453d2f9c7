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
    assert LN.select(torch.bfloat16, "gfx950", word="fast", cols=128).row == "hip_gfx950"
    with pytest.raises(LN.Refusal):
        LN.select(torch.bfloat16, "gfx950", word="fast", cols=2048)


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
    with pytest.raises(PF.Unsupported) as e:
        PF.pack_triattn_weights(w_o=w, n_heads=4, head_dim=32, w_q=w, w_k=w, w_v=w, w_g=w, w_b=torch.randn(4, 128), b_o=torch.zeros(128))
    assert e.value.reason == "projection_bias"
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

"""The C ABI without a GPU: libfpf_hip.so loads, exports every entry point include/fpf_hip.h declares, reports its version,
and the ctypes argument blocks match the header's field order.  No compute call is made (there is no device here)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "fpf_hip.h")


def _declared():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|size_t|const char\*)\s+(fpf_\w+)\s*\(", txt, flags=re.M)))


def _structs():
    """{struct name: [field names in order]} parsed from the header's typedef blocks."""
    txt = open(HEADER).read()
    out = {}
    for body, name in re.findall(r"typedef struct \{(.*?)\}\s*(\w+);", txt, flags=re.S):
        fields = []
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        for ln in body.splitlines():
            ln = ln.strip()
            if not ln:
                continue
            decl = ln.rstrip(";").strip()
            m = re.match(r"(?:const\s+)?[\w]+\s*\*?\s*(.+)$", decl)
            for part in m.group(1).split(","):
                part = part.strip().lstrip("*").strip()
                fields.append(re.sub(r"\[.*\]", "", part))
        out[name] = fields
    return out


def test_header_declares_the_entry_points():
    d = _declared()
    for must in ("fpf_abi_version", "fpf_describe", "fpf_layernorm_fwd", "fpf_transition_fwd", "fpf_trimul_fwd", "fpf_trimul_workspace_bytes",
                 "fpf_triattn_fwd", "fpf_triattn_block_fwd", "fpf_triattn_block_workspace_bytes", "fpf_triattn_prologue_fwd",
                 "fpf_triattn_epilogue_fwd", "fpf_triattn_bias_fwd", "fpf_apb_fwd", "fpf_apb_bias_fwd"):
        assert must in d, must


def test_library_loads_and_exports_every_declared_symbol():
    from fpf_hip import _lib as L
    if not os.path.exists(L.LIB_PATH):
        pytest.fail("libfpf_hip.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(L.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(L.ENTRY_POINTS) == _declared(), "ctypes binding and header disagree"
    assert L.lib().fpf_abi_version() == L.ABI_VERSION
    assert b"gfx950" in L.lib().fpf_describe()


def test_ctypes_blocks_follow_the_header_field_order():
    from fpf_hip import _lib as L
    st = _structs()
    pairs = {"FpfLnArgs": L.LnArgs, "FpfTransitionArgs": L.TransitionArgs, "FpfTrimulArgs": L.TrimulArgs, "FpfTriattnArgs": L.TriattnArgs,
             "FpfTriattnBlockArgs": L.TriattnBlockArgs, "FpfTriattnPrologueArgs": L.TriattnPrologueArgs,
             "FpfTriattnEpilogueArgs": L.TriattnEpilogueArgs, "FpfTriattnBiasArgs": L.TriattnBiasArgs, "FpfApbArgs": L.ApbArgs,
             "FpfApbBiasArgs": L.ApbBiasArgs}
    assert set(pairs) == set(st), sorted(st)
    for cname, py in pairs.items():
        assert [f[0] for f in py._fields_] == st[cname], cname


def test_workspace_queries_need_no_device():
    from fpf_hip import _lib as L
    lib = L.lib()
    # trimul: 3 channel-major bf16 planes of Np^2, Np = ceil(N / 128) * 128
    assert lib.fpf_trimul_workspace_bytes(1, 768, 128, 128, L.DT_BF16) >= 3 * 128 * 768 * 768 * 2
    assert lib.fpf_trimul_workspace_bytes(1, 100, 128, 128, L.DT_BF16) >= 3 * 128 * 128 * 128 * 2
    # tri-att block: q, k, v, o (H*D per pixel; the bf16 epilogue recomputes g) + fp32 bias (H per pixel); fp32 adds g
    need = lib.fpf_triattn_block_workspace_bytes(1, 768, 0, 128, 4, 32, L.DT_BF16)
    assert 4 * 768 * 768 * 128 * 2 + 768 * 768 * 4 * 4 <= need < 5 * 768 * 768 * 128 * 2
    assert lib.fpf_triattn_block_workspace_bytes(1, 768, 0, 128, 4, 32, L.DT_F32) >= 5 * 768 * 768 * 128 * 4
    # a row chunk holds the q / k / v / o of its rows only (plus the full bias)
    part = lib.fpf_triattn_block_workspace_bytes(1, 2048, 256, 128, 4, 32, L.DT_BF16)
    assert 4 * 256 * 2048 * 128 * 2 <= part < 4 * 300 * 2048 * 128 * 2 + 2048 * 2048 * 4 * 4 + 4096


def test_integration_stub_sends_the_header_version():
    """The ctypes stubs of the integration notes must not pin an ABI version other than the header's: every literal
    abi_version / fpf_abi_version() comparison there equals FPF_ABI_VERSION, which equals the binding's ABI_VERSION."""
    from fpf_hip import _lib as L
    hdr = int(re.search(r"#define FPF_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert hdr == L.ABI_VERSION
    txt = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    lits = [int(x) for x in re.findall(r"abi_version\s*=\s*(\d+)", txt)] + [int(x) for x in re.findall(r"fpf_abi_version\(\)\s*==\s*(\d+)", txt)]
    lits += [int(x) for x in re.findall(r"\((\d+) for this header\)", txt)]
    assert all(v == hdr for v in lits), lits
    assert "abi_version=ABI" in txt and "fpf_abi_version()" in txt


def test_version_mismatch_is_refused_before_any_launch():
    """A wrong abi_version is rejected by the argument gate (no device work is reached, so this runs without a GPU)."""
    from fpf_hip import _lib as L
    a = L.LnArgs(abi_version=L.ABI_VERSION + 1, dtype_in=L.DT_BF16, dtype_out=L.DT_BF16, cols=128, rows=4)
    with pytest.raises(L.LibError) as e:
        L.call("fpf_layernorm_fwd", a, None)
    assert e.value.kind == "version"
    a = L.TrimulArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, c_z=128, c_h=128, batch=1, n=8)
    with pytest.raises(L.LibError) as e:
        L.call("fpf_trimul_fwd", a, None)                  # NULL z / weights
    assert e.value.kind == "args"


def test_transition_pair_bias_gate_needs_no_device():
    """The transition's pair-bias fields are checked before any launch: w_z without a bias buffer (and the reverse), heads outside
    1 .. 32, rows that are not B N N pixels, an fp32 call (placeholder addresses: nothing is dereferenced)."""
    from fpf_hip import _lib as L
    p = 0x10000

    def args(**kw):
        base = dict(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, c=128, hidden=512, rows=2 * 8 * 8, x=p, out=p, w_a=p, w_b=p, w_o=p,
                    w_z=p, z_heads=4, pair_n=8, z_bias=p, z_bias_dtype=L.DT_F32)
        base.update(kw)
        return L.TransitionArgs(**base)
    for kw, kind, text in ((dict(z_bias=None), "args", "without z_bias"), (dict(w_z=None), "args", "without w_z"),
                           (dict(z_heads=33), "shape", "z_heads"), (dict(pair_n=7), "shape", "rows = B N N"),
                           (dict(z_bias_dtype=L.DT_U8), "dtype", "z_bias_dtype"), (dict(z_bias_ld=5), "shape", "z_bias_ld"),
                           (dict(dtype=L.DT_F32), "dtype", "bf16 transition")):
        with pytest.raises(L.LibError) as e:
            L.call("fpf_transition_fwd", args(**kw), None)
        assert e.value.kind == kind and text in e.value.msg, (kw, e.value.kind, e.value.msg)


def test_apb_refusals_need_no_device():
    """The attention-with-pair-bias gate refuses NULL operands and unserved head dims by name (nothing is launched)."""
    from fpf_hip import _lib as L
    a = L.ApbArgs(abi_version=L.ABI_VERSION, dtype=L.DT_F32, S=1, N=8, NK=8, H=2, D=24)
    with pytest.raises(L.LibError) as e:
        L.call("fpf_apb_fwd", a, None)
    assert e.value.kind == "args"
    b = L.ApbBiasArgs(abi_version=L.ABI_VERSION, dtype=L.DT_F32, B=1, N=8, C=128, H=16)
    with pytest.raises(L.LibError) as e:
        L.call("fpf_apb_bias_fwd", b, None)
    assert e.value.kind == "args"


def test_build_reads_kernel_resource_usage_and_refuses_vgpr_spills():
    """The build reads the compiler's kernel-resource-usage remarks per kernel (a kernel that spills vector registers is refused:
    its reloads' waits would drain the transfers in flight inside its loops)."""
    from fpf_hip import _build
    txt = ("a.hip:1:1: remark: Function Name: _Zk1 [-Rpass-analysis=kernel-resource-usage]\n"
           "a.hip:1:1: remark:     VGPRs: 200 [-Rpass-analysis=kernel-resource-usage]\n"
           "a.hip:1:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]\n"
           "a.hip:1:1: remark:     Occupancy [waves/SIMD]: 2 [-Rpass-analysis=kernel-resource-usage]\n"
           "a.hip:9:1: remark: Function Name: _Zk2 [-Rpass-analysis=kernel-resource-usage]\n"
           "a.hip:9:1: remark:     VGPRs Spill: 12 [-Rpass-analysis=kernel-resource-usage]\n")
    ru = _build.resource_usage(txt)
    assert ru == {"_Zk1": {"VGPRs": 200, "VGPRs Spill": 0, "Occupancy": 2}, "_Zk2": {"VGPRs Spill": 12}}
    # a register array in scratch memory (no counted spill) is refused too; a few SGPR-spill slots are not
    usage = dict(ru, _Zk3={"VGPRs Spill": 0, "ScratchSize": 1088}, _Zk4={"VGPRs Spill": 0, "SGPRs Spill": 53, "ScratchSize": 36})
    assert _build.refused(usage) == ["_Zk2", "_Zk3"]

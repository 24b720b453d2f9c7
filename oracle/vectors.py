"""The reference's golden-vector input generators, restated -- TEST INFRASTRUCTURE ONLY.

Each generator reproduces the reference's inputs byte for byte; the tests check every generated tensor against the SHA-256
digest the reference recorded in its manifest (copied into tests/golden/*.json by tests/golden/make_fixtures.py), so a
generator that drifts fails by name instead of comparing against the wrong operands.

    triattn_inputs     common/opt_core/opt_core/kernels/triattn/triattn_native/pkg/v11/testvectors/cases.py:109-149
    trimul_inputs      common/opt_core/opt_core/kernels/trimul/native/pkg/v5/python/trimul_native/vectors.py:1-24 (recipe
                       closed_form_v1), :117-188
    transition_inputs  common/opt_core/opt_core/kernels/transition/flash_sm90a/cells/vectors.py:18-34
"""
import hashlib

import numpy as np
import torch

PAD_FRAC = 0.07
BIAS_SCALE = 0.5
_DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def tensor_sha256(t):
    """SHA-256 of a tensor's values in logical row-major order (bool as one byte per element)."""
    c = t.detach().contiguous().cpu()
    if c.dtype == torch.bool:
        c = c.to(torch.uint8)
    return hashlib.sha256(c.reshape(-1).view(torch.uint8).numpy().tobytes()).hexdigest()


# ------------------------------------------------------------------------------------------------------------ triangle attention
def triattn_inputs(case):
    """{q, k, v, bias, mask, scale} for a triattn case record (keys N S H D B dtype mask bias layout seed).  Drawn from one CPU
    generator seeded 1000003*seed + 131*N + S: q, k, v (randn fp32 -> dtype), bias randn*0.5 ([B,1,H,S,S]; 'bf16x' rounds it
    through the 16-bit dtype and back to fp32, 'bias16' keeps the 16-bit tensor), then for 'prefixvar' one kept length per row
    drawn in [S - 3 round(0.07 S), S] with row 0 full ('prefix': one length S - round(0.07 S) for every row).  Layout
    'endstrided' draws q/k/v as [B,S,H,N,D] storage and hands the dim-1 <-> dim-3 transposed views."""
    seed, N, S = int(case["seed"]), int(case["N"]), int(case["S"])
    B, H, D = int(case.get("B", 1)), int(case.get("H", 4)), int(case.get("D", 32))
    dt = _DT[case.get("dtype", "bf16")]
    g = torch.Generator("cpu").manual_seed(1000003 * seed + 131 * N + S)

    def rnd(*shape, s=1.0):
        return torch.randn(*shape, generator=g, dtype=torch.float32) * s

    layout = case.get("layout", "start")
    if layout == "start":
        q, k, v = (rnd(B, N, H, S, D).to(dt) for _ in range(3))
    elif layout == "endstrided":
        q, k, v = (rnd(B, S, H, N, D).to(dt) for _ in range(3))
    else:
        raise ValueError(layout)
    bias = rnd(B, 1, H, S, S, s=BIAS_SCALE)
    bk = case.get("bias", "bf16x")
    if bk in ("bf16x", "bias16"):
        bias = bias.to(dt).float()
        if bk == "bias16":
            bias = bias.to(dt)
    elif bk != "fp32":
        raise ValueError(bk)
    npad = int(round(PAD_FRAC * S))
    mk = case.get("mask", "none")
    if mk == "prefix":
        L = torch.full((B, N), max(S - npad, 1), dtype=torch.int64)
    elif mk == "prefixvar":
        L = torch.randint(max(1, S - 3 * npad), S + 1, (B, N), generator=g, dtype=torch.int64)
        L[:, 0] = S
    elif mk == "none":
        L = None
    else:
        raise ValueError(mk)
    mask = None
    if L is not None:
        mask = (torch.arange(S)[None, None, :] < L[:, :, None])[:, :, None, None, :].contiguous()
    if layout == "endstrided":
        q, k, v = (t.transpose(1, 3) for t in (q, k, v))
    return {"q": q, "k": k, "v": v, "bias": bias, "mask": mask, "scale": float(D) ** -0.5}


# ------------------------------------------------------------------------------------------------------------ triangle multiplication
_M32 = 0xFFFFFFFF


def _mix(a):
    a = a & _M32
    for _ in range(3):
        a = a ^ (a >> 16)
        a = (a * 0x45D9F3B) & _M32
    return a ^ (a >> 16)


def _h(i, j, c, salt):
    return _mix((i * 2654435 + j * 40503 + c * 97 + salt * 7919) & _M32)


def trimul_inputs(case, weight_salt=0):
    """(z, mask or None, weights dict) for a trimul case record (keys c_z c_hidden n batch form mask), recipe closed_form_v1:
    integer hashes of the indices scaled by powers of two, exact in the target dtype.  Weights are bf16 for form 'bf16' and fp32
    for 'f32z'; z likewise."""
    cz, ch, n, B = int(case["c_z"]), int(case["c_hidden"]), int(case["n"]), int(case.get("batch", 1))
    i = torch.arange(n, dtype=torch.int64).view(n, 1, 1)
    j = torch.arange(n, dtype=torch.int64).view(1, n, 1)
    c = torch.arange(cz, dtype=torch.int64).view(1, 1, cz)
    zs = []
    for b in range(B):
        r = 100 + (7 * i + 3 * j) % 155
        kk = _h(i, j, c, 1 + 16 * b) % (2 * r + 1) - r
        zb = kk.to(torch.float32) / 128.0
        if case["form"] == "f32z":
            k2 = _h(i, j, c, 2 + 16 * b) % 129 - 64
            zb = zb + k2.to(torch.float32) * (2.0 ** -16)
        else:
            zb = zb.to(torch.bfloat16)
        zs.append(zb)
    z = zs[0] if B == 1 else torch.stack(zs, 0)
    mask = None
    if case["mask"] == "tail3":
        m = torch.ones(n, n, dtype=torch.float32)
        m[n - 3:, :] = 0
        m[:, n - 3:] = 0
        mask = m if B == 1 else m.unsqueeze(0).expand(B, n, n).contiguous()
    elif case["mask"] != "none":
        raise ValueError(case["mask"])

    def mat(rows, cols, salt):
        o = torch.arange(rows, dtype=torch.int64).view(rows, 1)
        q = torch.arange(cols, dtype=torch.int64).view(1, cols)
        return ((_h(o, q, 0, salt) % 255) - 127).to(torch.float32) / 2048.0

    def vec(length, salt, base, scale):
        o = torch.arange(length, dtype=torch.int64)
        return base + ((_h(o, 0, 0, salt) % 65) - 32).to(torch.float32) / scale
    ws = 1000 * int(weight_salt)
    w = {"ln_in_w": vec(cz, 21 + ws, 1.0, 256.0), "ln_in_b": vec(cz, 22 + ws, 0.0, 512.0),
         "w_ag": mat(ch, cz, 11 + ws), "w_ap": mat(ch, cz, 12 + ws), "w_bg": mat(ch, cz, 13 + ws), "w_bp": mat(ch, cz, 14 + ws),
         "ln_out_w": vec(ch, 23 + ws, 1.0, 256.0), "ln_out_b": vec(ch, 24 + ws, 0.0, 512.0),
         "w_o": mat(cz, ch, 15 + ws), "w_og": mat(cz, cz, 16 + ws)}
    if case["form"] == "bf16":
        w = {k_: v_.to(torch.bfloat16) for k_, v_ in w.items()}
    return z, mask, w


def trimul_weights_digest(w):
    """The manifest's combined weights digest: sha256 of the concatenated per-tensor hex digests in sorted key order."""
    return hashlib.sha256("".join(tensor_sha256(w[k]) for k in sorted(w)).encode()).hexdigest()


# ------------------------------------------------------------------------------------------------------------ transition
def transition_inputs(rows, seed, c_in=256, hidden=1024):
    """(z, w_a, w_b, w_o, ln_w, ln_b): numpy RandomState(seed) float32 normals in the order z (x4), w_a, w_b (x c^-1/2),
    w_o (x hidden^-1/2) -> bf16 (round to nearest even); ln_w = 1 + 0.1 N(0,1), ln_b = 0.05 N(0,1) in fp32."""
    rs = np.random.RandomState(seed)

    def t(shape, scale):
        return torch.from_numpy((rs.standard_normal(shape) * scale).astype(np.float32)).to(torch.bfloat16)
    z = t((rows, c_in), 4.0)
    wa = t((hidden, c_in), c_in ** -0.5)
    wb = t((hidden, c_in), c_in ** -0.5)
    wo = t((c_in, hidden), hidden ** -0.5)
    ln_w = 1.0 + 0.1 * torch.from_numpy(rs.standard_normal(c_in).astype(np.float32))
    ln_b = 0.05 * torch.from_numpy(rs.standard_normal(c_in).astype(np.float32))
    return z, wa, wb, wo, ln_w, ln_b

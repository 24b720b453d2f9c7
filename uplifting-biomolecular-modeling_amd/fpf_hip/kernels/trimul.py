"""Triangle-multiplication face, served by libfpf_hip's ``fpf_trimul_fwd`` (K1 planes -> batched MFMA contraction -> K3).

Mirrors common/opt_core/opt_core/kernels/trimul/__init__.py: the op (:3-11), ``WEIGHT_KEYS`` (:171), ``Refusal`` (:188),
``select`` (:835) and ``triangle_multiplication(z, mask=None, *, direction, weights, word=None, selection=None, residual=False,
cache=None, eps=1e-5, ...)`` (:1982).  ``cache`` (a dict the caller holds per weight set) keeps the packed weights and the
workspace between calls; keys carry the weight tensors' identity, so a dict shared across modules re-packs rather than
serving another module's pack.  ``out`` may be ``z`` itself when ``residual=True`` (K3 reads each pixel before writing it).
"""
import torch

from .. import _face as F
from .. import _lib as L
from .. import cells as CELLS

Refusal, Selection = F.Refusal, F.Selection
WEIGHT_KEYS = ("ln_in_w", "ln_in_b", "w_ag", "w_ap", "w_bg", "w_bp", "ln_out_w", "ln_out_b", "w_o", "w_og")
_DIRS = {"outgoing": "outgoing", "out": "outgoing", "incoming": "incoming", "in": "incoming"}


def direction_word(direction):
    d = _DIRS.get(str(direction))
    if d is None:
        raise ValueError("direction must be outgoing | incoming (got %r)" % (direction,))
    return d


def select(arch, dtype, c_z, c_hidden, n_tokens, direction="outgoing", *, word):
    """Pure: the row serving a TriMul call of this class, or Refusal by name."""
    d = direction_word(direction)
    sel = F.resolve(word, F.dtype_word(dtype), arch, "trimul",
                    cell=CELLS.trimul_key(F.dtype_word(dtype), c_z, c_hidden, n_tokens, "out" if d == "outgoing" else "in"))
    if sel.row == F.ROW_FAST and (c_z, c_hidden) != (128, 128):
        raise Refusal("shape:c%dx%d" % (c_z, c_hidden), sel.row, F.ROW_F32, "the bf16 kernels serve c_z = c_hidden = 128")
    if sel.row == F.ROW_F32 and (c_z > 128 or c_hidden > 128):
        raise Refusal("shape:c%dx%d" % (c_z, c_hidden), sel.row, F.ROW_STOCK, "the fp32 kernels serve c_z, c_hidden <= 128")
    return sel


def _pack(weights, dtype, device, cache):
    key = ("_pack", str(device), dtype) + tuple(id(weights[k]) for k in WEIGHT_KEYS)
    p = cache.get(key)
    if p is None:
        missing = [k for k in WEIGHT_KEYS if weights.get(k) is None]
        if missing:
            raise Refusal("weights_missing:" + ",".join(missing), None, F.ROW_STOCK)
        with torch.no_grad():
            p = {}
            for k in WEIGHT_KEYS:
                t = weights[k].detach().to(device)
                p[k] = t.float().contiguous() if k.startswith("ln_") else t.to(dtype).contiguous()
        for k_ in [k_ for k_ in cache if isinstance(k_, tuple) and k_[:1] == ("_pack",)]:
            del cache[k_]
        cache[key] = p
    return p


def triangle_multiplication(z, mask=None, *, direction, weights, word=None, selection=None, residual=False, cache=None, eps=1e-5,
                            out=None, **_unused):
    """Returns the update (or z + update when ``residual``) in z's dtype; Refusal by name before any launch."""
    cache = {} if cache is None else cache
    z4 = z if z.dim() == 4 else z.unsqueeze(0)
    B, N, N2, Cz = z4.shape
    if N != N2:
        raise ValueError("z must be [B,N,N,c] or [N,N,c] (got %s)" % (tuple(z.shape),))
    d = direction_word(direction)
    Ch = int(weights["w_ap"].shape[0])
    sel = selection or select(F.device_word(z), z.dtype, Cz, Ch, N, d, word=word)
    if not z4.is_contiguous():
        raise Refusal("stride", sel.row, F.ROW_STOCK, "z must be contiguous")
    p = _pack(weights, z.dtype, z.device, cache)
    m = None
    if mask is not None:
        m = mask if mask.dim() == 3 else mask.unsqueeze(0)
        if tuple(m.shape) != (B, N, N):
            raise Refusal("mask_shape", sel.row, F.ROW_STOCK, str(tuple(mask.shape)))
        m = m.to(device=z.device, dtype=torch.float32).contiguous()
    if out is None:
        out = torch.empty_like(z)
    elif out.shape != z.shape or out.dtype != z.dtype or not out.is_contiguous():
        raise Refusal("out", sel.row, F.ROW_STOCK, "out must be contiguous with z's shape and dtype")
    if out.data_ptr() == z.data_ptr() and not residual:
        raise Refusal("out_aliases_z", sel.row, F.ROW_STOCK, "out may alias z only for the residual form")
    dt = L.DT_BF16 if z.dtype == torch.bfloat16 else L.DT_F32
    need = L.lib().fpf_trimul_workspace_bytes(B, N, Cz, Ch, dt)
    wkey = ("_ws", str(z.device))
    ws = cache.get(wkey)
    if ws is None or ws.numel() < need:
        ws = cache[wkey] = torch.empty(need, dtype=torch.uint8, device=z.device)
    a = L.TrimulArgs(abi_version=L.ABI_VERSION, dtype=dt, c_z=Cz, c_h=Ch, batch=B, n=N, z=L.ptr(z4), out=L.ptr(out), mask=L.ptr(m),
                     ln_in_w=L.ptr(p["ln_in_w"]), ln_in_b=L.ptr(p["ln_in_b"]), ln_out_w=L.ptr(p["ln_out_w"]), ln_out_b=L.ptr(p["ln_out_b"]),
                     w_ag=L.ptr(p["w_ag"]), w_ap=L.ptr(p["w_ap"]), w_bg=L.ptr(p["w_bg"]), w_bp=L.ptr(p["w_bp"]), w_o=L.ptr(p["w_o"]),
                     w_og=L.ptr(p["w_og"]), outgoing=1 if d == "outgoing" else 0, residual=1 if residual else 0, eps=float(eps),
                     workspace=L.ptr(ws), workspace_bytes=ws.numel())
    L.call("fpf_trimul_fwd", a, L.stream_ptr(z.device))
    cache["_last"] = sel
    return out

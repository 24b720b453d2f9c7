"""Shared pieces of the provider faces: the row / tier-word vocabulary, ``Refusal``, ``Selection`` and the device word.

Rows served by this package (one per arithmetic class; the reference's faces name their rows the same way):
    hip_gfx950      bf16 operands, fp32 accumulation / statistics / softmax (MFMA 32x32x16 bf16)        class fast
    hip_gfx950_f32  fp32 operands and fp32 arithmetic throughout                                        class exact (fp32 path)
    stock           the caller's own stock statement (named; never run here)                            class stock

Words (the reference's vocabulary, common/opt_core/opt_core/kernels/triattn/__init__.py:25-36):
    fast / big      -> hip_gfx950 for bf16 inputs, hip_gfx950_f32 for fp32 inputs
    exact           -> hip_gfx950_f32 for fp32 inputs; bf16 inputs are refused by name (fallback 'stock'): the fp32 path is this
                       package's exact tier, and a bf16 call has no vouched bitwise row here.  Where the measured cell table
                       (fpf_hip/cells) names the stock statement as the cell's exact row (it measured faster than
                       hip_gfx950_f32), 'exact' is refused by name with fallback 'stock', as the reference's exact rule does
    a row name      -> exactly that row, or a Refusal naming the fallback row
A refusal is raised before anything is launched and never after a kernel started (the reference's rule,
triattn/__init__.py:129-136).
"""
from collections import namedtuple

ROW_FAST = "hip_gfx950"
ROW_F32 = "hip_gfx950_f32"
ROW_STOCK = "stock"
ROW_NAMES = (ROW_FAST, ROW_F32, ROW_STOCK)
TIER_WORDS = ("fast", "exact", "big")
ARCH = "gfx950"

Selection = namedtuple("Selection", "row word cell cls reason")


class Refusal(RuntimeError):
    """A row cannot serve this call: ``kind`` = the refusal word, ``row`` = the row asked for, ``fallback`` = the row to bind
    instead.  Raised before any launch."""

    def __init__(self, kind, row=None, fallback=ROW_STOCK, detail=""):
        self.kind, self.row, self.fallback, self.detail = kind, row, fallback, detail
        RuntimeError.__init__(self, "row %r refused: %s%s%s" % (row, kind, (" (%s)" % detail) if detail else "",
                                                                   ("; bind instead: %r" % fallback) if fallback else ""))


_ARCH_BY_DEVICE = {}


def device_word(t):
    """'gfx950' for an MI355X tensor (the arch name without feature suffixes), 'cpu' for a host tensor.  Memoised per device
    index (the property query is a runtime call)."""
    if not t.is_cuda:
        return "cpu"
    idx = t.device.index
    w = _ARCH_BY_DEVICE.get(idx)
    if w is None:
        import torch
        w = _ARCH_BY_DEVICE[idx] = torch.cuda.get_device_properties(t.device).gcnArchName.split(":")[0]
    return w


_RESOLVED = {}


def resolve(word, dtype_word, arch, face, cell=None):
    """Pure selection shared by the faces: (word, 'bf16' | 'fp32', arch) -> Selection, or Refusal by name.  Memoised per
    argument tuple like the reference's selection memo (refusals are re-raised from the memo)."""
    key = (word, dtype_word, arch, face, cell)
    hit = _RESOLVED.get(key)
    if hit is None:
        try:
            hit = _resolve(word, dtype_word, arch, face, cell)
        except Refusal as r:
            hit = r
        _RESOLVED[key] = hit
    if isinstance(hit, Refusal):
        raise Refusal(hit.kind, hit.row, hit.fallback, hit.detail)
    return hit


def _resolve(word, dtype_word, arch, face, cell):
    if word is None:
        raise ValueError("word is required (a row name or one of %s)" % (TIER_WORDS,))
    w = str(word)
    if w == ROW_STOCK:
        raise Refusal("stock_is_the_callers_statement", ROW_STOCK, None, "%s: the stock row is the caller's own call" % face)
    if arch != ARCH:
        raise Refusal("arch:%s" % arch, w, ROW_STOCK, "%s rows are gfx950 kernels" % face)
    if w in ("fast", "big"):
        row = ROW_FAST if dtype_word == "bf16" else ROW_F32
    elif w == "exact":
        if dtype_word != "fp32":
            raise Refusal("exact:%s_input" % dtype_word, w, ROW_STOCK, "the exact tier is the fp32 path (pass fp32 operands)")
        row = ROW_F32
    elif w in (ROW_FAST, ROW_F32):
        row = w
    else:
        raise Refusal("unknown_word:%s" % w, w, ROW_STOCK)
    want = "bf16" if row == ROW_FAST else "fp32"
    if dtype_word != want:
        raise Refusal("dtype:%s" % dtype_word, row, ROW_F32 if row == ROW_FAST else ROW_FAST, "row %s takes %s operands" % (row, want))
    cls = "fast" if row == ROW_FAST else "exact"
    reason = "%s: %s -> %s (%s, %s)" % (face, w, row, dtype_word, arch)
    if cell:
        from . import cells
        m = cells.lookup(face, cell)
        if w == "exact" and m is not None and m.get("exact") == ROW_STOCK:
            raise Refusal("exact:stock_faster", w, ROW_STOCK, "%s: the fp32 torch statement measured x%.2f faster than %s in cell %s"
                          % (face, 1.0 / max(m.get("x_stock", {}).get(row, 1.0), 1e-9), row, cell))
        if m is not None and row in m.get("ms", {}):
            reason += "; cell %s: %.3f ms measured, x%.2f over the torch statement" % (cell, m["ms"][row], m.get("x_stock", {}).get(row, float("nan")))
    return Selection(row, w, cell, cls, reason)


def dtype_word(dtype):
    import torch
    if dtype == torch.bfloat16:
        return "bf16"
    if dtype == torch.float32:
        return "fp32"
    return str(dtype).replace("torch.", "")

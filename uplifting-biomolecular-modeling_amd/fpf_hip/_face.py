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
# compute capability -> arch word: ROCm torch reports an MI355X (gfx950) as capability (9, 5)
CC_ARCH = {(9, 5): ARCH}


def norm_cc(cc):
    """(major, minor) from a capability given as a tuple / list, "9.5", 9.5, "sm_95" or "sm95" (the reference's forms,
    common/opt_core/opt_core/kernels/triattn/__init__.py:197-206)."""
    if isinstance(cc, (tuple, list)):
        return int(cc[0]), int(cc[1])
    s = str(cc).strip()
    if s.startswith("sm"):
        s = (s[3:] if s.startswith("sm_") else s[2:]).rstrip("a")
        return int(s[:-1]), int(s[-1])
    major, _, minor = s.partition(".")
    return int(major), int(minor or 0)


def arch_word(cc):
    """The device word a row is keyed by, from whatever the caller names the device with: a capability (tuple, "9.5", "sm_95"),
    an arch name ("gfx950", "gfx950:sramecc+:xnack-"), a tensor, or a torch.device.  (9, 5) is gfx950; any other capability
    gives "cc<M>.<m>", which no row of this package serves (refused by name)."""
    import torch
    if isinstance(cc, torch.Tensor):
        return device_word(cc)
    if isinstance(cc, torch.device):
        if cc.type != "cuda":
            return "cpu"
        idx = cc.index if cc.index is not None else torch.cuda.current_device()
        w = _ARCH_BY_DEVICE.get(idx)
        if w is None:
            w = _ARCH_BY_DEVICE[idx] = torch.cuda.get_device_properties(idx).gcnArchName.split(":")[0]
        return w
    if isinstance(cc, str) and cc.strip().startswith("gfx"):
        return cc.strip().split(":")[0]
    if cc is None:
        raise ValueError("cc is required (a capability such as (9, 5) or '9.5', an arch name such as 'gfx950', or a device)")
    M, m = norm_cc(cc)
    return CC_ARCH.get((M, m), "cc%d.%d" % (M, m))


def dtype_of(dtype):
    """'bf16' / 'fp32' / 'fp16' (or the dtype's own name) from a torch dtype or one of the reference's dtype words."""
    s = str(dtype).replace("torch.", "").strip().lower()
    return {"bfloat16": "bf16", "bf16": "bf16", "float32": "fp32", "float": "fp32", "f32": "fp32", "fp32": "fp32", "float16": "fp16",
            "half": "fp16", "fp16": "fp16"}.get(s, s)


def check_device(face, row, dev, **tensors):
    """Refusal by name unless every given tensor (None skipped) lives on ``dev``: a host pointer handed to a kernel is a device
    memory fault, so this runs before any launch."""
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise Refusal("device:%s" % name, row, ROW_STOCK, "%s: %s is on %s, the call runs on %s" % (face, name, t.device, dev))


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
    return dtype_of(dtype)


def no_config(config, row):
    """The kernels' launch geometry is fixed per shape class: an explicit launch setting (the reference passes Triton configs
    through) is refused by name rather than ignored."""
    if config:
        raise Refusal("config:fixed_launch", row, row, "launch settings %s are not tunable on this row" % (dict(config),))


def word_base(word):
    """``row@<config>`` words name a launch setting the reference's Triton rows take; this package's rows have none."""
    w = str(word)
    if "@" in w:
        base, _, cfg = w.partition("@")
        raise Refusal("config_word:%s" % cfg, base, base, "word %r: the launch geometry of this row is fixed" % w)
    return w


def narrow(sel, word, prefer, exclude=None):
    """Apply the caller's candidate narrowing to a resolved Selection: ``prefer`` (rows, in order) restricts a tier word's
    candidates, ``exclude`` steps aside from rows; the row this package resolved must survive both, else Refusal by name."""
    if prefer and str(word) in TIER_WORDS and sel.row not in [str(p).split("@")[0] for p in prefer]:
        raise Refusal("prefer_excludes:%s" % sel.row, word, str(list(prefer)[0]), "prefer=%s" % (tuple(prefer),))
    if exclude and sel.row in [str(e) for e in exclude]:
        raise Refusal("excluded:%s" % sel.row, word, ROW_STOCK, "exclude=%s" % (tuple(exclude),))
    return sel


# ---------------------------------------------------------------------------------------------------------------- scratch
_SCRATCH = {}
_CAPTURED = []      # outgrown buffers that a captured call used: a graph replays with their addresses, so they stay allocated


def scratch(device, nbytes, kind="ws"):
    """One grow-only device buffer per (device, stream, kind), shared by every call of every face on that stream: a call uses
    its workspace only between its own launches on the current stream, so the next call on the same stream may reuse it, and
    a stack of layers holds ONE workspace sized by its largest call instead of one per layer.  Calls on other streams get
    their own buffers.  ``kind`` separates buffers one call needs at the same time (the chunked triangle attention holds a
    workspace and a full bias).

    Graph capture: a buffer handed to a call while its stream is capturing is marked, and when a later, larger call outgrows
    it, the marked buffer is kept allocated (not returned to torch's caching allocator), so a graph that recorded its address
    never replays into memory torch has handed to another tensor.  ``reserve_scratch`` sizes the buffer up front instead, so
    that no captured call sees a buffer that is later outgrown; ``release_scratch`` drops everything, marked buffers included,
    and must not run while such a graph is still replayed."""
    import torch
    dev = torch.device(device)
    key = (str(dev), torch.cuda.current_stream(dev).cuda_stream if dev.type == "cuda" else 0, kind)
    t = _SCRATCH.get(key)
    if t is None or t.numel() < nbytes:
        old = _SCRATCH.pop(key, None)
        if old is not None and getattr(old, "_fpf_captured", False):
            _CAPTURED.append(old)
        del old, t                                           # an unmarked buffer goes back to the caching allocator first
        t = _SCRATCH[key] = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)
    if dev.type == "cuda" and not getattr(t, "_fpf_captured", False) and torch.cuda.is_current_stream_capturing():
        t._fpf_captured = True
    return t


def reserve_scratch(device, nbytes, kind="ws"):
    """Size the current stream's shared buffer of ``kind`` to at least ``nbytes`` now (before capturing a graph whose calls
    should never see it outgrown)."""
    return scratch(device, nbytes, kind)


def scratch_bytes(device=None):
    """Bytes held by the shared scratch buffers (of one device, or all)."""
    return sum(t.numel() for k, t in _SCRATCH.items() if device is None or k[0] == str(device))


def release_scratch():
    """Drop every shared scratch buffer, the outgrown ones a captured call used included (their memory returns to torch's caching
    allocator): no graph that captured a call of these faces may be replayed afterwards."""
    _SCRATCH.clear()
    del _CAPTURED[:]

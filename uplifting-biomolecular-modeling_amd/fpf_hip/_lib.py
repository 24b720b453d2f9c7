"""ctypes binding of libfpf_hip.so (include/fpf_hip.h).  The argument blocks mirror the header field for field; ``call``
maps a non-zero return into :class:`LibError` (code + the library's one-line message) -- nothing has been launched then.

torch is imported BEFORE the library is opened: torch carries its own HIP runtime (soname libamdhip64.so.7) and the
library's dependency on that soname must resolve to the copy torch already mapped, so one process holds one runtime.
"""
import ctypes as C
import os

import torch  # noqa: F401  (must precede the dlopen below: see the module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfpf_hip.so")
ABI_VERSION = 13
DT_BF16, DT_F32, DT_U8, DT_F32Z_BF16 = 1, 2, 3, 4
TRIMUL_NOALLOC_SCRATCH_BYTES = 50331648          # include/fpf_hip.h FPF_TRIMUL_NOALLOC_SCRATCH_BYTES
ERRORS = {1: "version", 2: "args", 3: "shape", 4: "dtype", 5: "align", 6: "workspace", 7: "launch"}

i32, i64, f32, vp, sz = C.c_int32, C.c_int64, C.c_float, C.c_void_p, C.c_size_t


class LnArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype_in", i32), ("dtype_out", i32), ("cols", i32), ("rows", i64), ("x", vp),
                ("x_row_stride", i64), ("y", vp), ("y_row_stride", i64), ("gamma", vp), ("beta", vp), ("eps", f32)]


class TransitionArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("c", i32), ("hidden", i32), ("rows", i64), ("x", vp), ("out", vp),
                ("ln_w", vp), ("ln_b", vp), ("eps", f32), ("w_a", vp), ("w_b", vp), ("w_o", vp), ("row_mask", vp), ("residual", i32),
                ("x_ln", vp), ("w_z", vp), ("z_ln_w", vp), ("z_ln_b", vp), ("z_eps", f32), ("z_heads", i32), ("pair_n", i64), ("z_bias", vp),
                ("z_bias_dtype", i32), ("z_bias_ld", i64)]


class TrimulArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("c_z", i32), ("c_h", i32), ("batch", i64), ("n", i64), ("z", vp), ("out", vp),
                ("mask", vp), ("ln_in_w", vp), ("ln_in_b", vp), ("ln_out_w", vp), ("ln_out_b", vp), ("w_ag", vp), ("w_ap", vp),
                ("w_bg", vp), ("w_bp", vp), ("w_o", vp), ("w_og", vp), ("outgoing", i32), ("residual", i32), ("eps", f32),
                ("workspace", vp), ("workspace_bytes", sz), ("row0", i64), ("rows", i64), ("fixed_in", vp)]


class TriattnArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("B", i64), ("N", i64), ("H", i64), ("S", i64), ("D", i64),
                ("q", vp), ("k", vp), ("v", vp), ("q_stride", i64 * 5), ("k_stride", i64 * 5), ("v_stride", i64 * 5), ("v_layout", i32),
                ("bias", vp), ("bias_dtype", i32), ("bias_stride", i64 * 4), ("mask", vp), ("mask_dtype", i32),
                ("mask_stride", i64 * 3), ("out", vp), ("out_stride", i64 * 5), ("scale", f32), ("keep", vp),
                ("workspace", vp), ("workspace_bytes", sz)]


class TriattnBlockArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("B", i64), ("N", i64), ("C", i32), ("H", i32), ("D", i32), ("z", vp),
                ("mask", vp), ("mask_dtype", i32), ("ln_w", vp), ("ln_b", vp), ("eps", f32), ("w_qkvg", vp), ("w_b", vp), ("w_o", vp),
                ("ending", i32), ("residual", i32), ("out", vp), ("scale", f32), ("workspace", vp), ("workspace_bytes", sz),
                ("row0", i64), ("rows", i64), ("bias_in", vp), ("mask_frame", i32), ("b_g", vp), ("b_o", vp), ("x_ln", vp)]


class TriattnBiasArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("B", i64), ("N", i64), ("C", i32), ("H", i32), ("D", i32), ("z", vp), ("ln_w", vp),
                ("ln_b", vp), ("eps", f32), ("w_qkvg", vp), ("w_b", vp), ("ending", i32), ("bias", vp)]


class TriattnPrologueArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("B", i64), ("N", i64), ("C", i32), ("H", i32), ("D", i32), ("z", vp), ("ln_w", vp),
                ("ln_b", vp), ("eps", f32), ("w_qkvg", vp), ("w_b", vp), ("ending", i32), ("q", vp), ("k", vp), ("v", vp), ("v_ld", i64),
                ("g", vp), ("bias", vp), ("b_g", vp), ("x_ln", vp)]


class TriattnEpilogueArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("B", i64), ("N", i64), ("C", i32), ("H", i32), ("D", i32), ("o", vp), ("g", vp),
                ("w_o", vp), ("ending", i32), ("residual", i32), ("out", vp), ("b_o", vp)]


class ApbArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("S", i64), ("N", i64), ("NK", i64), ("H", i64), ("D", i64), ("q", vp), ("k", vp),
                ("v", vp), ("q_stride", i64 * 4), ("k_stride", i64 * 4), ("v_stride", i64 * 4), ("gate", vp), ("gate_stride", i64 * 4),
                ("bias", vp), ("bias_dtype", i32), ("bias_stride", i64 * 4), ("key_mask", vp), ("mask_dtype", i32),
                ("mask_stride", i64 * 2), ("out", vp), ("out_stride", i64 * 4), ("scale", f32)]


class ApbBiasArgs(C.Structure):
    _fields_ = [("abi_version", i32), ("dtype", i32), ("B", i64), ("N", i64), ("C", i32), ("H", i32), ("z", vp), ("ln_w", vp), ("ln_b", vp),
                ("eps", f32), ("w_z", vp), ("bias", vp), ("bias_dtype", i32), ("bias_ld", i64)]


ENTRY_POINTS = {                     # name -> (argtypes, restype); every symbol include/fpf_hip.h declares
    "fpf_abi_version": ([], C.c_int),
    "fpf_describe": ([], C.c_char_p),
    "fpf_layernorm_fwd": ([C.POINTER(LnArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_transition_fwd": ([C.POINTER(TransitionArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_trimul_workspace_bytes": ([i64, i64, i32, i32, i32], sz),
    "fpf_trimul_fwd": ([C.POINTER(TrimulArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_trimul_fwd_noalloc": ([C.POINTER(TrimulArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_trimul_fixed_fwd": ([C.POINTER(TrimulArgs), vp, vp, C.c_char_p, sz], C.c_int),
    "fpf_trimul_fixed_bytes": ([i64, i64, i32, i32], sz),
    "fpf_trimul_rows_workspace_bytes": ([i64, i64, i64, i32, i32], sz),
    "fpf_trimul_channels_fwd": ([C.POINTER(TrimulArgs), i64, vp, C.c_char_p, sz], C.c_int),
    "fpf_trimul_channels_workspace_bytes": ([i64, i64, i64, i32, i32], sz),
    "fpf_triattn_fwd": ([C.POINTER(TriattnArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_triattn_block_workspace_bytes": ([i64, i64, i64, i32, i32, i32, i32], sz),
    "fpf_triattn_bias_bytes": ([i64, i64, i32, i32], sz),
    "fpf_triattn_stage_bytes": ([i64, i64, i64, i64, i64, i32], sz),
    "fpf_triattn_workspace_bytes": ([i64, i64, i64, i64, i32], sz),
    "fpf_triattn_bias_fwd": ([C.POINTER(TriattnBiasArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_triattn_block_fwd": ([C.POINTER(TriattnBlockArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_triattn_prologue_fwd": ([C.POINTER(TriattnPrologueArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_triattn_epilogue_fwd": ([C.POINTER(TriattnEpilogueArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_apb_fwd": ([C.POINTER(ApbArgs), vp, C.c_char_p, sz], C.c_int),
    "fpf_apb_bias_fwd": ([C.POINTER(ApbBiasArgs), vp, C.c_char_p, sz], C.c_int),
}


class LibError(RuntimeError):
    """The library refused a call before launching anything: ``kind`` (version | args | shape | dtype | align | workspace |
    launch) and the library's message."""

    def __init__(self, entry, code, msg):
        self.entry, self.code, self.kind, self.msg = entry, code, ERRORS.get(code, str(code)), msg
        RuntimeError.__init__(self, "%s -> %s: %s" % (entry, self.kind, msg))


class LibraryMissing(RuntimeError):
    """libfpf_hip.so is not built (run __graft_entry__.build() or python -m fpf_hip._build)."""


_LIB = None


def lib():
    """The opened library (opened once per process).  Raises LibraryMissing when the .so is absent -- the faces never fall
    back to another implementation."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing("%s is not built: run __graft_entry__.build()" % LIB_PATH)
        L = C.CDLL(LIB_PATH)
        for name, (argt, rest) in ENTRY_POINTS.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.argtypes = argt
            fn.restype = rest
        if L.fpf_abi_version() != ABI_VERSION:
            raise LibraryMissing("libfpf_hip.so abi %d != %d: rebuild" % (L.fpf_abi_version(), ABI_VERSION))
        _LIB = L
    return _LIB


def hip_runtimes_mapped():
    """Paths of every libamdhip64 mapped into this process (one expected)."""
    out = set()
    try:
        with open("/proc/self/maps") as f:
            for ln in f:
                if "libamdhip64" in ln:
                    out.add(ln.split()[-1])
    except OSError:
        pass
    return sorted(out)


def stream_ptr(device=None):
    """The raw hipStream_t of torch's current stream on ``device``."""
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def call(name, args, *rest):
    """Invoke an entry point ``name(&args, *rest, err, errlen)`` (``rest`` ends with the stream); raise LibError on refusal."""
    err = C.create_string_buffer(512)
    fn = getattr(lib(), name, None)
    if fn is None:
        raise LibraryMissing("libfpf_hip.so does not export %s: rebuild" % name)
    rc = fn(C.byref(args), *rest, err, 512)
    if rc != 0:
        raise LibError(name, rc, err.value.decode(errors="replace"))


def ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())

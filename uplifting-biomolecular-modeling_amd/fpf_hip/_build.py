"""Build libfpf_hip.so in-tree with hipcc for gfx950 (no cmake, no JIT cache): each csrc/*.hip compiles to an object in
parallel, then one link.  ``python -m fpf_hip._build`` or ``__graft_entry__.build()``."""
import concurrent.futures as cf
import glob
import json
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
CSRC = os.path.join(PKG_ROOT, "csrc")
REPO = os.path.dirname(PKG_ROOT)
INCLUDE = os.path.join(REPO, "include")
LIB = os.path.join(HERE, "libfpf_hip.so")
OBJ_DIR = os.path.join(PKG_ROOT, "_build")
ARCH = os.environ.get("FPF_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
# packed fp32 VALU forms are disabled: the kernels' fp32 arithmetic must stay on the scalar-lane VALU forms
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I" + INCLUDE, "-I" + CSRC, "-Wno-unused-result", "-Rpass-analysis=kernel-resource-usage"]
def refused(usage):
    """Kernels the build refuses: a VGPR spill, or more scratch than a few SGPR-spill slots (a register array the compiler
    placed in scratch memory, e.g. one captured by a lambda it did not inline).  Either reloads registers from memory inside
    the kernel's loops, and each reload's wait drains the loads and DMA transfers in flight."""
    return sorted(k for k, v in usage.items() if v.get("VGPRs Spill", 0) or v.get("ScratchSize", 0) > SCRATCH_LIMIT)


SCRATCH_LIMIT = 64          # bytes per lane: the SGPR-spill slots some kernels keep; a spilled register array is far larger
_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|VGPRs Spill|SGPRs Spill|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]):\s*(\S+)")


def resource_usage(text):
    """{kernel: {field: value}} from the compiler's kernel-resource-usage remarks (one block per kernel, starting at its name)."""
    out, cur = {}, None
    for m in _REMARK.finditer(text):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[key.split(" [")[0]] = int(val) if val.isdigit() else val
    return out


def _compile(src):
    obj = os.path.join(OBJ_DIR, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC] + FLAGS + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    res = resource_usage(r.stdout)
    out = "\n".join(ln for ln in r.stdout.splitlines() if "packed-fp32-ops" not in ln and "kernel-resource-usage" not in ln
                    and not ln.lstrip().startswith(("|", "^")) and not re.match(r"^\s*\d+\s*\|", ln))
    if r.returncode != 0:
        raise RuntimeError("hipcc failed on %s:\n%s" % (src, out))
    return obj, out, res


def build(verbose=False):
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError("no HIP sources under %s" % CSRC)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        res = list(ex.map(_compile, srcs))
    usage = {}
    for obj, out, ru in res:
        usage.update(ru)
        if verbose and out.strip():
            print(out)
    spilled = refused(usage)
    if spilled:
        raise RuntimeError("kernels spill vector registers to scratch: %s" % ", ".join("%s (%s)" % (k, usage[k]) for k in spilled))
    with open(os.path.join(OBJ_DIR, "resources.json"), "w") as f:
        json.dump(usage, f, indent=1, sort_keys=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + [o for o, _, _ in res]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

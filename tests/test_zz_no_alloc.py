"""fpf_trimul_fwd_noalloc: triangle multiplication with the library's static per-device scratch instead of a caller workspace,
called through the C ABI and compared with fpf_trimul_fwd (caller workspace) on the same inputs: bitwise equal (the same
kernels on the same operands), on two calls in a row, the second on a smaller input, so stale scratch contents from the
first call would show.  Plus the refusals that need no launch (a caller workspace, a size beyond the scratch)."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
KEYS = ("ln_in_w", "ln_in_b", "w_ag", "w_ap", "w_bg", "w_bp", "ln_out_w", "ln_out_b", "w_o", "w_og")


def _case(N, seed, masked):
    g = torch.Generator().manual_seed(seed)
    w = {k: (torch.randn(128, 128, generator=g) / 128 ** 0.5).to(torch.bfloat16).to(DEV) for k in ("w_ag", "w_ap", "w_bg", "w_bp", "w_o", "w_og")}
    w.update(ln_in_w=(1 + 0.1 * torch.randn(128, generator=g)).to(DEV), ln_in_b=(0.1 * torch.randn(128, generator=g)).to(DEV),
             ln_out_w=(1 + 0.1 * torch.randn(128, generator=g)).to(DEV), ln_out_b=(0.1 * torch.randn(128, generator=g)).to(DEV))
    z = torch.randn(1, N, N, 128, generator=g).to(torch.bfloat16).to(DEV)
    mask = None
    if masked:
        mask = torch.ones(1, N, N)
        mask[:, N - 9:, :] = 0
        mask[:, :, :3] = 0
        mask = mask.to(DEV)
    return z, mask, w


def _args(z, mask, w, out, outgoing, residual, ws=None):
    from fpf_hip import _lib as L
    N = int(z.shape[1])
    return L.TrimulArgs(abi_version=L.ABI_VERSION, dtype=L.DT_BF16, c_z=128, c_h=128, batch=1, n=N, z=L.ptr(z), out=L.ptr(out), mask=L.ptr(mask),
                        ln_in_w=L.ptr(w["ln_in_w"]), ln_in_b=L.ptr(w["ln_in_b"]), ln_out_w=L.ptr(w["ln_out_w"]), ln_out_b=L.ptr(w["ln_out_b"]),
                        w_ag=L.ptr(w["w_ag"]), w_ap=L.ptr(w["w_ap"]), w_bg=L.ptr(w["w_bg"]), w_bp=L.ptr(w["w_bp"]), w_o=L.ptr(w["w_o"]),
                        w_og=L.ptr(w["w_og"]), outgoing=int(outgoing), residual=int(residual), eps=1e-5, workspace=L.ptr(ws),
                        workspace_bytes=0 if ws is None else ws.numel())


def _both(N, seed, masked, outgoing, residual):
    """(out of fpf_trimul_fwd_noalloc, out of fpf_trimul_fwd) on one input."""
    from fpf_hip import _lib as L
    z, mask, w = _case(N, seed, masked)
    st = L.stream_ptr(DEV)
    out_na = torch.empty_like(z)
    print("[noalloc] N=%d outgoing=%s residual=%s masked=%s" % (N, outgoing, residual, masked), flush=True)
    L.call("fpf_trimul_fwd_noalloc", _args(z, mask, w, out_na, outgoing, residual), st)
    ws = torch.empty(L.lib().fpf_trimul_workspace_bytes(1, N, 128, 128, L.DT_BF16), dtype=torch.uint8, device=DEV)
    out_ws = torch.empty_like(z)
    L.call("fpf_trimul_fwd", _args(z, mask, w, out_ws, outgoing, residual, ws), st)
    torch.cuda.synchronize()
    return out_na, out_ws, z


def test_noalloc_equals_the_workspace_entry_on_two_calls_second_smaller():
    a1, b1, z1 = _both(256, 1, True, True, False)                 # the largest size the scratch holds
    assert torch.equal(a1, b1), "N=256: max diff %.3e" % (a1.float() - b1.float()).abs().max().item()
    assert torch.count_nonzero(a1) > 0
    a2, b2, z2 = _both(150, 2, False, False, True)                # smaller, incoming, residual: stale planes must not leak
    assert torch.equal(a2, b2), "N=150: max diff %.3e" % (a2.float() - b2.float()).abs().max().item()
    assert not torch.equal(a2, z2)


def test_noalloc_refusals_launch_nothing():
    from fpf_hip import _lib as L
    z, mask, w = _case(257, 3, False)                             # N = 257: 113 MB of planes, above the 48 MiB scratch
    out = torch.empty_like(z)
    with pytest.raises(L.LibError) as e:
        L.call("fpf_trimul_fwd_noalloc", _args(z, mask, w, out, True, False), L.stream_ptr(DEV))
    assert e.value.kind == "workspace"
    z, mask, w = _case(64, 4, False)
    ws = torch.empty(L.lib().fpf_trimul_workspace_bytes(1, 64, 128, 128, L.DT_BF16), dtype=torch.uint8, device=DEV)
    out = torch.zeros_like(z)
    with pytest.raises(L.LibError) as e:
        L.call("fpf_trimul_fwd_noalloc", _args(z, mask, w, out, True, False, ws), L.stream_ptr(DEV))
    assert e.value.kind == "args"
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0
    assert L.TRIMUL_NOALLOC_SCRATCH_BYTES == 3 * 128 * 256 * 256 * 2


def test_noalloc_on_a_side_stream_of_the_current_device():
    """The entry checks that the caller's stream belongs to the current device (the scratch address is per device; a stream of
    another device is refused before any launch).  A side stream of the current device passes the check and gives the same bits as
    the null-stream call; on a one-GPU box the refusal itself cannot be provoked."""
    from fpf_hip import _lib as L
    z, mask, w = _case(96, 5, True)
    out0, out1 = torch.empty_like(z), torch.empty_like(z)
    L.call("fpf_trimul_fwd_noalloc", _args(z, mask, w, out0, True, True), L.stream_ptr(DEV))
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(side):
        L.call("fpf_trimul_fwd_noalloc", _args(z, mask, w, out1, True, True), ctypes.c_void_p(side.cuda_stream))
    side.synchronize()
    assert torch.equal(out0, out1)

"""Measures the MI355X cell table (MI355X_CELLS.json next to this file) on the GPU box:

    python -m fpf_hip.cells.make_cells [--sizes 256,400,...] [--reps 5]

For every bucket size N and dtype (bf16 -> row hip_gfx950, fp32 -> row hip_gfx950_f32) it times this package's row and the
torch statement of the same op (the same dtype, on the same device: what the reference's tables call the stock op, here
written out in torch because the reference's stock libraries do not exist on this platform), median of ``reps`` calls
after one warm-up, with HIP events.  Shapes: triangle attention B = 1, H = 4, D = 32, S = N rows and keys, fp32 bias, mask
all ones; triangle multiplication B = 1, c_z = c_hidden = 128, both directions, mask all ones; transition c = 128, 4x
hidden, N^2 rows.  Inputs ~ N(0, 1), weights ~ N(0, 1/fan_in), seed 0.  Each timing follows at least 30 ms of untimed calls
(the torch statements: one call when a single call takes longer).

A cell's `fast` is this package's bf16 row; its `exact` follows the reference's exact rule (TRIATTN_CELLS.json
`exact_rule`): the fp32 row where it measured at least as fast as the fp32 torch statement, else "stock" -- the caller's own
statement, which the `exact` word then names as the row to bind.
"""
import argparse
import json
import os
import statistics
import sys
import time

import torch
import torch.nn.functional as Fn

from . import BUCKETS, CC, TABLE, transition_key, triattn_key, trimul_key
from .. import _face as F


def _median_ms(fn, reps, warm_s=0.03):
    """Median of ``reps`` timed calls after at least ``warm_s`` seconds of untimed calls (the first ~10 ms of a kernel stream
    after host-side set-up run slower than the steady state a stack of layers sees)."""
    fn()
    torch.cuda.synchronize()
    t0 = time.time()
    while time.time() - t0 < warm_s:
        fn()
        torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        ts.append(s.elapsed_time(e))
    return statistics.median(ts)


def _stock_triattn(q, k, v, bias, scale, rows=32):
    """softmax(scale q k^T + bias) v per pair row, in chunks of ``rows`` rows (the scores of all rows do not fit at large N)."""
    out = torch.empty_like(q)
    for n0 in range(0, q.shape[1], rows):
        qs, ks, vs = q[:, n0:n0 + rows], k[:, n0:n0 + rows], v[:, n0:n0 + rows]
        s = torch.matmul(qs, ks.transpose(-1, -2).contiguous()).float() * scale + bias.float()
        out[:, n0:n0 + rows] = torch.matmul(torch.softmax(s, dim=-1).to(q.dtype), vs)
    return out


def _stock_trimul(z, w, outgoing):
    x = Fn.layer_norm(z, (z.shape[-1],), w["ln_in_w"].to(z.dtype), w["ln_in_b"].to(z.dtype))
    a = torch.sigmoid(x @ w["w_ag"].t()) * (x @ w["w_ap"].t())
    b = torch.sigmoid(x @ w["w_bg"].t()) * (x @ w["w_bp"].t())
    if outgoing:                                                   # X[i,j,c] = sum_k a[i,k,c] b[j,k,c]
        X = torch.matmul(a.permute(0, 3, 1, 2).contiguous(), b.permute(0, 3, 2, 1).contiguous())
    else:                                                          # X[i,j,c] = sum_k a[k,i,c] b[k,j,c]
        X = torch.matmul(a.permute(0, 3, 2, 1).contiguous(), b.permute(0, 3, 1, 2).contiguous())
    X = X.permute(0, 2, 3, 1)
    y = Fn.layer_norm(X, (X.shape[-1],), w["ln_out_w"].to(z.dtype), w["ln_out_b"].to(z.dtype)) @ w["w_o"].t()
    return torch.sigmoid(x @ w["w_og"].t()) * y


def _stock_transition(x, w_a, w_b, w_o):
    n = Fn.layer_norm(x, (x.shape[-1],))
    return (Fn.silu(n @ w_a.t()) * (n @ w_b.t())) @ w_o.t()


def measure(sizes, reps, dev):
    from ..kernels import transition as TR
    from ..kernels import triattn as TA
    from ..kernels import trimul as TM
    gpu = torch.cuda.get_device_properties(dev)
    stack = "%s:torch%s" % (gpu.gcnArchName.split(":")[0], torch.__version__)
    g = torch.Generator().manual_seed(0)
    out = {}
    rows = {"hip_gfx950": "bf16 operands, fp32 accumulation / softmax / statistics (MFMA 32x32x16 bf16)",
            "hip_gfx950_f32": "fp32 operands and arithmetic throughout"}
    for face in ("triattn", "trimul", "transition"):
        out[face] = {"schema": "mi355x_cells/v1: the %s column for capability %s; key grammar in fpf_hip/cells/__init__.py" % (face, CC),
                     "stack": stack, "rows": rows, "buckets": {"sizes": list(sizes), "rule": "smallest listed size >= n_tokens; above the "
                     "largest the largest cell serves (measured = false)"}, "cells": {}}

    def put(face, key, row, ms_row, ms_stock):
        c = out[face]["cells"].setdefault(key, {"fast": None, "exact": None, "ms": {}, "stock_ms": None, "x_stock": {}})
        c["ms"][row] = round(ms_row, 4)
        c["stock_ms"] = round(ms_stock, 4)
        c["x_stock"][row] = round(ms_stock / ms_row, 2)
        if row == F.ROW_FAST:
            c["fast"] = row
        else:                                                      # the reference's exact rule: the exact-class row where it
            c["exact"] = row if ms_stock >= ms_row else F.ROW_STOCK   # measured >= x1.00 over the stock op, else the stock op

    for N in sizes:
        # each row is named directly (a tier word would resolve through the table being rebuilt)
        for dt, word, row in ((torch.bfloat16, F.ROW_FAST, F.ROW_FAST), (torch.float32, F.ROW_F32, F.ROW_F32)):
            dw = F.dtype_word(dt)
            # triangle attention op
            shp = (1, N, 4, N, 32)
            q, k, v = (torch.randn(shp, generator=g).to(dt).to(dev) for _ in range(3))
            bias = torch.randn(1, 1, 4, N, N, generator=g).to(dev)
            t_row = _median_ms(lambda: TA.triangle_attention(q, k, v, bias, None, word=word), reps)
            t_st = _median_ms(lambda: _stock_triattn(q, k, v, bias, 32 ** -0.5), max(1, reps // 2))
            put("triattn", triattn_key(dw, 32, 4, N), row, t_row, t_st)
            del q, k, v, bias
            # triangle multiplication, both directions
            z = torch.randn(1, N, N, 128, generator=g).to(dt).to(dev)
            w = {kk: (torch.randn(128, 128, generator=g) / 128 ** 0.5).to(dt).to(dev) for kk in ("w_ag", "w_ap", "w_bg", "w_bp", "w_o", "w_og")}
            w.update(ln_in_w=torch.ones(128, device=dev), ln_in_b=torch.zeros(128, device=dev),
                     ln_out_w=torch.ones(128, device=dev), ln_out_b=torch.zeros(128, device=dev))
            for d in ("out", "in"):
                cache = {}
                t_row = _median_ms(lambda: TM.triangle_multiplication(z, None, direction=d, weights=w, word=word, cache=cache), reps)
                t_st = _median_ms(lambda: _stock_trimul(z, w, d == "out"), max(1, reps // 2))
                put("trimul", trimul_key(dw, 128, 128, N, d), row, t_row, t_st)
            # transition (c = 128, 4x), the pair tensor's N^2 rows
            wa, wb = ((torch.randn(512, 128, generator=g) / 128 ** 0.5).to(dt).to(dev) for _ in range(2))
            wo = (torch.randn(128, 512, generator=g) / 512 ** 0.5).to(dt).to(dev)
            W = TR.pack(w_a=wa, w_b=wb, w_o=wo)
            t_row = _median_ms(lambda: TR.transition(z, W, word=word), reps)
            t_st = _median_ms(lambda: _stock_transition(z, wa, wb, wo), max(1, reps // 2))
            put("transition", transition_key(dw, 128, 4, N), row, t_row, t_st)
            del z, w, W
            torch.cuda.empty_cache()
            print("[cells] N=%d %s done" % (N, dw), flush=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--sizes", default=",".join(str(b) for b in BUCKETS))
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--out", default=TABLE)
    a = ap.parse_args()
    if not torch.cuda.is_available():
        print("make_cells measures on the GPU: no device here", file=sys.stderr)
        sys.exit(2)
    t0 = time.time()
    tab = measure([int(s) for s in a.sizes.split(",")], a.reps, torch.device("cuda:0"))
    tab["_meta"] = {"generated_by": "python -m fpf_hip.cells.make_cells --sizes %s --reps %d" % (a.sizes, a.reps),
                    "seconds": round(time.time() - t0, 1)}
    with open(a.out, "w") as f:
        json.dump(tab, f, indent=1, sort_keys=True)
    print("wrote", a.out, flush=True)


if __name__ == "__main__":
    main()

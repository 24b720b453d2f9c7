"""Write the golden fixtures under tests/golden/ from the DATA files the reference's own tests hold.

Run in the build container only (the reference tree is not present on the GPU box):

    python tests/golden/make_fixtures.py [--ref /root/reference]

Reads (as data; .pt files with torch.load(weights_only=True), JSON with the json module -- no reference module is imported):
    common/opt_core/opt_core/kernels/triattn/triattn_native/pkg/v11/testvectors/manifest.json and <id>.ref_rows.pt
        (the fp64 reference of pair row 0, stored fp32, per case)
    common/opt_core/opt_core/kernels/trimul/native/pkg/v5/testvectors/manifest.json and witness/<id>.<cls>.pt
        (input digests, the kernels' recorded error vs fp64, full H100/A100 outputs of the N = 32 witness cases)
    common/opt_core/opt_core/kernels/transition/flash_sm90a/cells/vectors.json and expected_M{8,333}.bf16
        (H100 stock bf16-autocast bytes of the c = 256 transition, residual form)
Writes: triattn_cases.json + triattn_ref_<id>.npy, trimul_cases.json + trimul_witness_<id>.<cls>.npy (bf16 bits as uint16),
transition_vectors.json + transition_expected_M{8,333}.bf16.
"""
import argparse
import json
import os
import shutil

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
TRIATTN_DIR = "common/opt_core/opt_core/kernels/triattn/triattn_native/pkg/v11/testvectors"
TRIMUL_DIR = "common/opt_core/opt_core/kernels/trimul/native/pkg/v5/testvectors"
TRANSITION_DIR = "common/opt_core/opt_core/kernels/transition/flash_sm90a/cells"

TRIATTN_IDS = ("s256_none", "s256_prefix", "n256_s256_none", "s384_endstrided", "s512_prefixvar", "a80_s400_prefixvar",
               "a80_d16_s512_prefix", "a80_b2_s400_prefix", "a80_h8_s800_prefixvar")
TRIMUL_IDS = ("c128x128_n32_out_bf16_res1_mtail3_fast", "c64x128_n32_out_bf16_res1_mtail3_fast",
              "c128x128_n256_out_bf16_res0_mnone_fast", "c128x128_n403_in_bf16_res1_mtail3_fast",
              "c128x128_n400_out_f32z_res1_mnone_fast", "c128x128_n256_b2_out_bf16_res0_mtail3_fast",
              "c128x128_n256_in_bf16_res0_mnone_fast")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    a = ap.parse_args()
    # --- triangle attention
    src = os.path.join(a.ref, TRIATTN_DIR)
    man = json.load(open(os.path.join(src, "manifest.json")))
    keep = []
    for c in man["cases"]:
        if c["id"] not in TRIATTN_IDS:
            continue
        rows = torch.load(os.path.join(src, c["ref"]["file"]), weights_only=True)
        np.save(os.path.join(HERE, "triattn_ref_%s.npy" % c["id"]), rows.numpy().astype(np.float32))
        keep.append({k: c[k] for k in ("id", "N", "S", "H", "D", "B", "dtype", "mask", "bias", "layout", "seed", "cc",
                                       "inputs_sha256", "err_vs_fp64", "out_shape")})
    json.dump({"source": TRIATTN_DIR + "/manifest.json", "ref_rows": "pair row 0 of the fp64 reference, stored fp32",
               "cases": keep}, open(os.path.join(HERE, "triattn_cases.json"), "w"), indent=1)
    # --- triangle multiplication
    src = os.path.join(a.ref, TRIMUL_DIR)
    man = json.load(open(os.path.join(src, "manifest.json")))
    keep = []
    for c in man["cases"]:
        if c["id"] not in TRIMUL_IDS:
            continue
        rec = {k: c[k] for k in ("id", "c_z", "c_hidden", "n", "batch", "direction", "form", "residual", "mask", "variant",
                                 "inputs_sha256", "witness")}
        rec["expected"] = {cls: {k: v for k, v in e.items() if k in ("dtype", "numerics", "shape", "sha256")}
                           for cls, e in c["expected"].items() if "numerics" in e}
        if c.get("witness"):
            for cls in ("sm90", "sm80"):
                p = os.path.join(src, "witness", "%s.%s.pt" % (c["id"], cls))
                if os.path.exists(p):
                    t = torch.load(p, weights_only=True)
                    np.save(os.path.join(HERE, "trimul_witness_%s.%s.npy" % (c["id"], cls)),
                            t.contiguous().view(torch.int16).numpy().view(np.uint16))
        keep.append(rec)
    json.dump({"source": TRIMUL_DIR + "/manifest.json", "recipe": man["recipe"], "cases": keep},
              open(os.path.join(HERE, "trimul_cases.json"), "w"), indent=1)
    # --- transition
    src = os.path.join(a.ref, TRANSITION_DIR)
    vec = json.load(open(os.path.join(src, "vectors.json")))
    json.dump(vec, open(os.path.join(HERE, "transition_vectors.json"), "w"), indent=1)
    for nm in ("expected_M8.bf16", "expected_M333.bf16"):
        shutil.copyfile(os.path.join(src, nm), os.path.join(HERE, "transition_" + nm))
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()

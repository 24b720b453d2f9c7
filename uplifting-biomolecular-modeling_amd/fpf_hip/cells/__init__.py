"""The MI355X column of the reference's cell tables: measured rows per (dtype, shape class, N bucket), so the tier words of
this package resolve to a named, measured cell the way the reference's faces do on their own parts.

Key grammars follow the reference's tables (common/opt_core/opt_core/kernels/triattn/TRIATTN_CELLS.json `schema`,
trimul/TRIMUL_CELLS.json `key_grammar`, transition/TRANSITION_CELLS.json `key_grammar`), with the capability column
"9.5" (torch.cuda.get_device_capability() on MI355X):

    triattn     9.5|<dtype>|D<head_dim>|H<heads>|N<=<bucket>|fwd
    trimul      9.5|<dtype>|C<c_z>|H<c_hidden>|N<=<bucket>|<in|out>|fwd
    transition  9.5|<dtype>|pair_c<c>_n<factor>|N<=<bucket>|eager|fwd

Bucket rule (the reference's, TRIATTN_CELLS.json `buckets.rule`): the smallest listed size >= the token count; above the
largest listed size the largest cell serves, marked measured = False.  The measured values live in MI355X_CELLS.json,
written on the GPU box by ``python -m fpf_hip.cells.make_cells`` (rows of this package against the torch statement of
the same op in the same dtype on the same device).
"""
import json
import os

CC = "9.5"
BUCKETS = (256, 400, 511, 800, 1200, 1536, 2048)
TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "MI355X_CELLS.json")


def bucket(n_tokens):
    """(bucket size, measured): the smallest listed size >= n_tokens, else the largest with measured = False."""
    for b in BUCKETS:
        if n_tokens <= b:
            return b, True
    return BUCKETS[-1], False


def triattn_key(dtype_word, head_dim, heads, n_tokens):
    return "%s|%s|D%d|H%d|N<=%d|fwd" % (CC, dtype_word, head_dim, heads, bucket(n_tokens)[0])


def trimul_key(dtype_word, c_z, c_hidden, n_tokens, direction):
    return "%s|%s|C%d|H%d|N<=%d|%s|fwd" % (CC, dtype_word, c_z, c_hidden, bucket(n_tokens)[0], direction)


def transition_key(dtype_word, c, factor, n_tokens):
    return "%s|%s|pair_c%d_n%d|N<=%d|eager|fwd" % (CC, dtype_word, c, factor, bucket(n_tokens)[0])


_LOADED = {}


def table():
    """The measured table ({face: {"cells": {key: cell}, ...}}), or {} when it has not been generated."""
    if "t" not in _LOADED:
        t = {}
        if os.path.exists(TABLE):
            with open(TABLE) as f:
                t = json.load(f)
        _LOADED["t"] = t
    return _LOADED["t"]


def lookup(face, key):
    """The measured cell for ``key`` of ``face`` ("triattn" | "trimul" | "transition"), or None."""
    return table().get(face, {}).get("cells", {}).get(key)

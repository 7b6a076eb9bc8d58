"""Shared test helpers: golden-case loading and bit comparisons."""

import glob
import json
import os

import numpy as np

from oracle import oracle as O
from oracle import tosa_reader as fb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")

FLOATS = ("FP32", "FP16", "BF16", "FP8E4M3", "FP8E5M2")


def case_dirs(kind="conformance"):
    if kind == "conformance":
        return sorted(glob.glob(os.path.join(GOLDEN, "conformance", "*", "*")))
    return sorted(glob.glob(os.path.join(GOLDEN, "networks", "*")))


def case_id(d):
    return os.path.relpath(d, GOLDEN)


class Case:
    def __init__(self, d):
        self.dir = d
        self.desc = json.load(open(os.path.join(d, "desc.json")))
        self.graph = open(os.path.join(d, self.desc["tosa_file"]), "rb").read()
        self.block = fb.main_block(self.graph)
        self.defs = {t.name: t for t in self.block.tensors}
        self.expected_failure = bool(self.desc.get("expected_failure", False))

    def inputs(self):
        """name -> (storage array, dtype)"""
        out = {}
        for n, f in zip(self.desc["ifm_name"], self.desc["ifm_file"]):
            dt = self.defs[n].dtype
            out[n] = (fb.load_npy(os.path.join(self.dir, f), dt), dt)
        return out

    def expected(self):
        out = {}
        for n, f in zip(self.desc["ofm_name"], self.desc["ofm_file"]):
            dt = self.defs[n].dtype
            out[n] = (fb.load_npy(os.path.join(self.dir, f), dt), dt)
        return out

    def tested_op(self):
        ops = [o.op for o in self.block.operators if o.op not in ("CONST", "CONST_SHAPE")]
        return ops[0] if len(ops) == 1 else None


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view({1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize]).reshape(-1)


def mismatches(got, exp, dtype):
    """Indices where `got` differs from `exp` bit for bit (any NaN equals any NaN)."""
    g = np.asarray(got).reshape(-1)
    e = np.asarray(exp).reshape(-1)
    if dtype in FLOATS:
        gb, eb = bits(g), bits(e)
        gv = O.decode(dtype, g.view(eb.dtype) if dtype != "FP32" else g)
        ev = O.decode(dtype, e.view(eb.dtype) if dtype != "FP32" else e)
        bad = ~((gb == eb) | (np.isnan(gv) & np.isnan(ev)))
    else:
        bad = g.astype(np.int64) != e.astype(np.int64)
    return np.nonzero(bad)[0]


def float_values(arr, dtype):
    return O.decode(dtype, np.asarray(arr)).astype(np.float64).reshape(-1)

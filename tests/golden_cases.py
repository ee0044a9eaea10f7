"""Loader for tests/golden/reference_golden.json (written from the reference's
own C code by tests/golden/make_golden.py)."""
import json
import os

import numpy as np

import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_golden.json")


def load():
    with open(GOLDEN) as f:
        return json.load(f)


def f32(bits):
    return np.array([bits], np.uint32).view(np.float32)[0]


def inputs(spec):
    """Regenerate a sampler case's row and history; checks the input digest."""
    row = synth.make_row(spec["kind"], spec["seed"], spec["V"])
    assert synth.digest(row) == spec["in_digest"], f"generator drift in case {spec['id']}"
    h = None
    if spec["n_hist"]:
        h = synth.history(spec["hist_seed"], 1, spec["n_hist"], spec["V"],
                          with_invalid=spec["invalid"])[0]
        if spec.get("dup") and spec["n_hist"] >= 8:
            h[5] = h[6] = h[7] = h[4]
        if spec.get("hot") is not None and spec["n_hist"] >= 2:
            h[-1] = spec["hot"]
            h[-2] = spec["hot"] + 1
    return row, h

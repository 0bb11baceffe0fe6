"""Loader for tests/golden/reference_vectors.json (vectors transcribed from the
reference's own tests; see tests/golden/make_reference_vectors.py)."""
import json
import os

import numpy as np

_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_vectors.json")


def cases(op=None):
    with open(_PATH) as f:
        data = json.load(f)["cases"]
    return [c for c in data if op is None or c["op"] == op]


def arr(c, name, dtype=np.float32):
    t = c["inputs"].get(name)
    if t is None:
        return None
    return np.asarray(t["data"], dtype=np.float64).reshape(t["shape"]).astype(dtype)


def conv_attrs(c):
    a = dict(c["attrs"])
    a.pop("kernel_shape", None)
    if c["op"] == "Conv1D":
        # Rank 1 is lowered onto the rank-2 kernel as [N,C,1,W], exactly as
        # the reference does (conv/conv_nd.rs:48-131).
        if "strides" in a:
            a["strides"] = [1] + a["strides"]
        if "dilations" in a:
            a["dilations"] = [1] + a["dilations"]
        if "pads" in a:
            a["pads"] = [0, a["pads"][0], 0, a["pads"][1]]
    return a


def conv_inputs(c):
    x, w, b = arr(c, "x"), arr(c, "w"), arr(c, "b")
    if c["op"] == "Conv1D":
        x = x.reshape(x.shape[0], x.shape[1], 1, x.shape[2])
        w = w.reshape(w.shape[0], w.shape[1], 1, w.shape[2])
    return x, w, b

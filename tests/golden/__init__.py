"""Frozen vectors written by make_golden.py (test data only)."""
import json
from pathlib import Path

import numpy as np


def load_golden():
    raw = json.loads(Path(__file__).with_name("golden.json").read_text())
    dq = [dict(name=c["name"], qtype=c["qtype"], n=c["n"], k=c["k"],
               blocks=np.frombuffer(bytes.fromhex(c["blocks"]), np.uint8),
               out=np.frombuffer(bytes.fromhex(c["out_f32"]), np.float32)) for c in raw["dequant"]]
    gv = [dict(name=c["name"], qtype=c["qtype"], n=c["n"], k=c["k"],
               blocks=np.frombuffer(bytes.fromhex(c["blocks"]), np.uint8),
               x=np.frombuffer(bytes.fromhex(c["x_f32"]), np.float32).reshape(1, c["k"]).copy(),
               y=np.frombuffer(bytes.fromhex(c["y_f64"]), np.float64).reshape(1, c["n"])) for c in raw["gemv"]]
    return {"dequant": dq, "gemv": gv}

"""The oracle still reproduces the frozen fixtures of tests/golden/."""
import numpy as np

import oracle
from tests.golden import load_golden
from tests import reference_np as ref


def test_oracle_reproduces_dequant_fixtures():
    for c in load_golden()["dequant"]:
        rc, y = oracle.dequant_tensor(c["qtype"], c["blocks"], c["n"] * c["k"])
        assert rc == 0
        assert np.array_equal(y.view(np.uint32), c["out"].view(np.uint32)), c["name"]
        # and the independent restatement agrees with the frozen vector
        assert np.array_equal(ref.DECODERS[c["qtype"]](c["blocks"]).view(np.uint32),
                              c["out"].view(np.uint32)), c["name"]


def test_oracle_reproduces_gemv_fixtures():
    for c in load_golden()["gemv"]:
        rc, wf = oracle.dequant_tensor(c["qtype"], c["blocks"], c["n"] * c["k"])
        y = oracle.linear_f64(c["x"], wf.reshape(c["n"], c["k"]))
        assert np.array_equal(y, c["y"]), c["name"]

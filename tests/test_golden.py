"""The committed golden vectors are reproduced by the oracle from their stored 16-bit inputs."""

import numpy as np
import pytest

from oracle import attention_oracle as orc
from tests.golden.make_golden import CASES, load


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    z = load(name)
    f64 = [z[key].double().numpy() for key in ("q", "k", "v", "do")]
    cu = orc.cu_seqlens_from_lengths(z["lengths"])
    o, lse = orc.attention_forward(f64[0], f64[1], f64[2], cu, float(z["scale"]))
    dq, dk, dv = orc.attention_backward(f64[0], f64[1], f64[2], o, lse, f64[3], cu,
                                        float(z["scale"]))
    for mine, key in ((o, "o"), (lse, "lse"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(mine, z[key], rtol=1e-6, atol=1e-6)
    assert z["q"].shape == (sum(z["lengths"]), int(z["hq"]), 128)

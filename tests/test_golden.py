"""The committed golden fixtures on the CPU: inputs regenerate bit-identically,
the oracle's output matches the fixture's float64 truth (within one bf16 ulp
for decode; for DiT, one ulp plus the P-to-bf16 rounding bound) and is
bit-identical to the output recorded when the fixture was made."""
import numpy as np
import pytest

import golden_cases as GC
import refs


@pytest.mark.parametrize("name", GC.NAMES)
def test_fixture_inputs_regenerate(name):
    case, truth, meta = GC.load(name)
    assert truth.ndim == 3 and np.all(np.isfinite(truth))


@pytest.mark.parametrize("name", GC.NAMES)
def test_oracle_matches_fixture(oracle, name):
    case, truth, meta = GC.load(name)
    _, ob = GC.MF.truth_and_oracle(name, case)
    got = refs.bits_to_f64(ob).reshape(truth.shape)
    err = np.abs(got - truth)
    bound = refs.bf16_ulp(truth)
    if GC.MF.SPECS[name]["kind"] == "dense":
        bound = bound + 2.0 ** -8 * refs.dense_weight_abs(case, 0)
    assert np.all(err <= bound), f"{name}: worst excess {np.max(err - bound):.3g}"
    assert GC.MF.digest(ob) == meta["oracle_digest"], f"{name}: oracle output changed since the fixture was made"
    tol = meta["tolerance"]
    assert err.max() <= tol["max_abs"] and err.mean() <= tol["mean_abs"]

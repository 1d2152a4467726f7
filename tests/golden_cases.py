"""Loads the committed golden fixtures (tests/golden/*.npz + fixtures.json)
and rebuilds each case: index arrays from the file, values from the oracle's
generator, checked against the stored digests."""
from __future__ import annotations

import json
import os
import sys

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)

import make_fixtures as MF  # noqa: E402

NAMES = list(MF.SPECS)


def index() -> dict:
    with open(os.path.join(GOLDEN, "fixtures.json")) as f:
        return json.load(f)


def load(name: str):
    """(case, truth f64 array, fixture metadata). Raises if the regenerated
    values do not match the digests the fixture was made with."""
    meta = index()[name]
    with np.load(os.path.join(GOLDEN, f"{name}.npz")) as z:
        arrays = {k: z[k] for k in z.files}
    case = MF.build(name, arrays if MF.SPECS[name]["kind"] != "dense" else None)
    got = MF.value_digests(name, case)
    if got != meta["digests"]:
        raise AssertionError(f"{name}: regenerated inputs differ from the fixture's digests")
    return case, arrays["truth"].astype(np.float64), meta

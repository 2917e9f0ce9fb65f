"""The CPU oracle against the committed golden fixtures (tests/golden, written by
tests/golden/make_fixtures.py): a change to the oracle that moves any recorded
result fails here."""
import os

import numpy as np
import pytest

import oracle
from golden.make_fixtures import STATE_CASES, TRACE_CASES, adam_case, state_case, trace_case

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name,config,ncell,tstop,mons", TRACE_CASES, ids=[c[0] for c in TRACE_CASES])
def test_oracle_traces_match_fixture(name, config, ncell, tstop, mons):
    ref = load(name)
    got = trace_case(config, ncell, tstop, mons)
    assert got["traces"].shape == ref["traces"].shape
    np.testing.assert_allclose(got["traces"], ref["traces"], rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(got["spike_gid"], ref["spike_gid"])
    np.testing.assert_allclose(got["spike_t"], ref["spike_t"], rtol=0, atol=1e-12)


@pytest.mark.parametrize("name,config,ncell,nstep", STATE_CASES, ids=[c[0] for c in STATE_CASES])
def test_oracle_state_matches_fixture(name, config, ncell, nstep):
    ref = load(name)
    got = state_case(config, ncell, nstep)
    for k in ref:
        np.testing.assert_allclose(got[k], ref[k], rtol=1e-12, atol=1e-14, err_msg=k)


def test_oracle_adam_matches_fixture():
    ref = load("adam_3steps")
    got = adam_case()
    for k in ref:
        np.testing.assert_allclose(got[k], ref[k], rtol=1e-15, atol=0, err_msg=k)


def test_fixtures_are_plain_arrays():
    for f in os.listdir(HERE):
        if f.endswith(".npz"):
            with np.load(os.path.join(HERE, f), allow_pickle=False) as z:
                for k in z.files:
                    assert z[k].dtype != object

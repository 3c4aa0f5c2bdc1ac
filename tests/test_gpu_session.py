"""The step-wise decode session of the persistent kernel alternates two
logit buffers and token slots between steps (the host-ring copy of step t
overlaps pass t): splits of the steps at odd and even boundaries, in both
reduction orders and with sampling, give the one-call decode's bits."""
import json
import os

import numpy as np
import pytest

from cis2amd import Cis2Model, artifacts

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", [0, 1])
def test_odd_splits_equal_one_call(mode):
    spec = artifacts.SPECS["smollm2-135m"]
    w = artifacts.Weights(spec, 20261201)
    prompt = artifacts.prompt_ids(20261201, spec.vocab, 32)
    m = Cis2Model(spec, w, max_pos=32 + 256, reduction_mode=mode)
    one = m.decode(prompt, 256)
    fx = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                     "model_fixtures.json")))
    ref = fx["smollm2-135m" if mode == 0 else "smollm2-135m-tree"]
    assert one["witness"] == ref["witness"]
    for splits in ([1, 255], [5, 11, 16, 224], [3, 3, 3, 247], [255, 1]):
        m.begin(prompt, 256)
        for n in splits:
            m.steps(n)
        r = m.end(256)
        assert r["witness"] == one["witness"], splits
        assert r["step_digests"] == one["step_digests"], splits
        assert np.array_equal(r["ids"], one["ids"]), splits
    m.set_sampling(3, 0.9, 20, 0.9)
    s_one = m.decode(prompt, 64)
    m.begin(prompt, 64)
    for n in (7, 1, 56):
        m.steps(n)
    s_parts = m.end(64)
    assert s_parts["witness"] == s_one["witness"]
    m.close()

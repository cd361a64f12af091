"""The self-check's comparisons reject what they must (CPU) and its cases pass on the GPU."""

from __future__ import annotations

import pytest
import torch

from jitengine_amd import selfcheck


def test_comparisons_reject_a_planted_difference():
    w = torch.linspace(-3, 3, 1000)
    selfcheck._close("same", w.to(torch.bfloat16), w)
    bad = w.clone()
    bad[500] += 0.1
    with pytest.raises(selfcheck.SelfCheckError, match="planted"):
        selfcheck._close("planted", bad.to(torch.bfloat16), w)
    with pytest.raises(selfcheck.SelfCheckError, match="cosine|err"):
        selfcheck._close("flipped", (-w).to(torch.bfloat16), w)
    selfcheck._equal("ids", torch.arange(8, dtype=torch.int32), torch.arange(8, dtype=torch.int32))
    with pytest.raises(selfcheck.SelfCheckError, match="ids"):
        selfcheck._equal("ids", torch.arange(8, dtype=torch.int32).flip(0), torch.arange(8, dtype=torch.int32))
    with pytest.raises(ValueError, match="GPU"):
        selfcheck.run("cpu")


@pytest.mark.gpu
def test_selfcheck_cases_pass_on_the_device():
    names = selfcheck.run("cuda", force=True)
    assert len(names) == len(selfcheck.CASES)
    assert selfcheck.run("cuda") == []  # once per device

"""Write-path staging of one loop group (residualquant_amd/group.py), after
DeferredKVGroup (src/residual_quantization/install_model.py:17-52): the
group keeps copies of its earlier loops' K/V and hands every record over on
its last loop."""

from __future__ import annotations

import pytest
import torch

from residualquant_amd import DeferredKVGroup
from residualquant_amd.layout import page_width

CONFIG = {"reference_mode": "anchor", "anchor_index": 2, "coefficient_method": "ls"}
RECORDS = ((2, 32), (2, 16), (4, 32))


def test_stage_keeps_copies_until_the_last_loop():
    group = DeferredKVGroup(CONFIG, RECORDS, 16)
    kv = [(torch.randn(5, 2, 128).to(torch.bfloat16), torch.randn(5, 2, 128).to(torch.bfloat16)) for _ in range(3)]
    originals = [(k.clone(), v.clone()) for k, v in kv]
    assert group.stage(*kv[0]) is None and group.stage(*kv[1]) is None
    kv[0][0].zero_()  # the group holds copies, not the caller's tensors
    records = group.stage(*kv[2])
    assert len(records) == 3 and group.pending == []
    for (k, v), (k0, v0) in zip(records[:2], originals[:2]):
        assert torch.equal(k, k0) and torch.equal(v, v0)
    assert records[2][0] is kv[2][0]  # the completing call borrows its input
    assert group.stage(*kv[0]) is None  # and the next group starts over


def test_single_record_group_hands_over_at_once():
    group = DeferredKVGroup(CONFIG | {"anchor_index": 0}, ((4, 32),), 16)
    k = torch.zeros(3, 1, 128, dtype=torch.bfloat16)
    assert group.stage(k, k) == [(k, k)]


def test_page_width_and_validation():
    group = DeferredKVGroup(CONFIG, RECORDS, 16)
    assert group.page_width(128) == page_width(128, RECORDS)
    with pytest.raises(ValueError, match="Unsupported reference"):
        DeferredKVGroup(CONFIG | {"reference_mode": "chain"}, RECORDS, 16)
    with pytest.raises(ValueError, match="anchor_index=0"):
        DeferredKVGroup(CONFIG | {"reference_mode": "adjacent"}, RECORDS, 16)
    with pytest.raises(ValueError, match="coefficient"):
        DeferredKVGroup(CONFIG | {"coefficient_method": "max"}, RECORDS, 16)
    with pytest.raises(ValueError, match="at least one record"):
        DeferredKVGroup(CONFIG, (), 16)

"""CPU: the Python op boundary keeps the reference's ValueError contract.

Every check here raises before any device work, so it runs without a GPU
(the reference's checks, sihc/models/sihc/sublayer_kernels.py:180-193, 235-243,
337-347, kernels.py:1770, 1792-1801, 2224-2227, 2345-2350, 2439-2442, 2536, and the
packed-layout test research/tests/test_sublayer_kernels.py:111-121).
"""
from __future__ import annotations

import pytest
import torch

from sihc_hip import blockwise_kernels as BK
from sihc_hip import event_ops as EV
from sihc_hip import indexed as IX
from sihc_hip import kernels as LK
from sihc_hip import sublayer_kernels as SK


def test_non_contiguous_carrier_is_rejected_with_packed_wording():
    x = torch.randn(1, 16, 16, 37)
    a = torch.randn(16, 37, 16)
    with pytest.raises(ValueError, match="contiguous|packed"):
        SK.sublayer_read(x.transpose(1, 2), a)


def test_prefix_slice_is_rejected_by_triangular():
    padded = torch.randn(2, 18, 37)
    bad = padded[:, 2:]
    assert not bad.is_contiguous()
    with pytest.raises(ValueError, match="contiguous|packed"):
        SK.sublayer_triangular(bad, [bad], torch.ones(1, 37))


def test_event_slot_and_grid_checks():
    x = torch.randn(2, 8, 8, 5)
    with pytest.raises(ValueError, match="1..32 events"):
        SK.sublayer_read(x, torch.randn(33, 5, 4))
    with pytest.raises(ValueError, match="4/16 spatial slots"):
        SK.sublayer_read(x, torch.randn(2, 5, 9))
    with pytest.raises(ValueError, match="square"):
        SK.sublayer_read(torch.randn(2, 8, 6, 5), torch.randn(2, 5, 4))
    with pytest.raises(ValueError, match="CUDA device and dtype"):
        SK.sublayer_read(x, torch.randn(2, 5, 4))  # CPU tensors are not accepted


def test_update_and_gamma_checks():
    # (The update-count check follows the device check, as in the reference, so it
    # is exercised by the GPU tests.)
    base = torch.randn(2, 16, 5)
    with pytest.raises(ValueError, match="active prefix"):
        SK.sublayer_triangular(base, [base], torch.ones(2, 5))
    with pytest.raises(ValueError, match="active updates"):
        SK.sublayer_triangular(base, [torch.randn(2, 16, 4)], torch.ones(1, 5))
    with pytest.raises(ValueError, match="workspace dtype or fp32"):
        SK.sublayer_triangular(base, [base], torch.ones(1, 5, dtype=torch.float64))


def test_blockwise_adapter_checks():
    x = torch.randn(2, 8, 8, 5)
    with pytest.raises(ValueError, match="8 or 12"):
        BK.blockwise_read(x, torch.randn(16, 5, 4))
    base = torch.randn(2, 16, 5)
    with pytest.raises(ValueError, match="1..11"):
        BK.blockwise_triangular(base, [base] * 12, torch.ones(12, 5))


def test_event_op_checks():
    x = torch.randn(2, 8, 8, 5)
    dz = torch.randn(2, 16, 5)
    with pytest.raises(ValueError, match="contiguous|packed"):
        EV.event_write_read(x.transpose(1, 2), dz, torch.randn(5, 4), torch.randn(5, 4))
    with pytest.raises(ValueError, match="update geometry"):
        EV.event_write_read(x, torch.randn(2, 15, 5), torch.randn(5, 4), torch.randn(5, 4))
    with pytest.raises(ValueError, match="CUDA device"):
        EV.event_write_read(x, dz, torch.randn(5, 4), torch.randn(5, 4))


def test_index_contract():
    idx = IX.group_index(3, grid=4, group=5, seed=1)
    assert idx.dtype == torch.int32 and idx.shape == (3, 16)
    for row in idx:
        assert sorted(row.tolist()) == list(range(16))
    # group structure: consecutive runs of 5 are ascending
    for row in idx.tolist():
        for i in range(0, 16, 5):
            assert row[i:i + 5] == sorted(row[i:i + 5])
    IX.check_index(idx, 3, 4, permutation=True)
    with pytest.raises(ValueError, match="permutations"):
        dup = idx.clone()
        dup[0, 1] = dup[0, 0]
        IX.check_index(dup, 3, 4, permutation=True)
    with pytest.raises(ValueError, match=r"\[0, 16\)"):
        bad = idx.clone()
        bad[1, 3] = 16
        IX.check_index(bad, 3, 4, permutation=False)
    with pytest.raises(ValueError, match="int32"):
        IX.check_index(idx.long(), 3, 4, permutation=False)
    # seeded: same seed, same assignment
    assert torch.equal(idx, IX.group_index(3, grid=4, group=5, seed=1))


def test_legacy_op_surface_and_shape_checks():
    # every reference op name is registered, one triangular op per prefix length
    assert len(LK.triangular_accumulate_b4_12_ptr_active_traceable_ops) == 11
    assert len(LK.triangular_accumulate_b4_8_ptr_active_traceable_ops) == 7
    for name in ("all_base_b4_12_split_traceable", "all_base_b4_8_split_traceable", "all_base_p8_12_split_traceable",
                 "all_base_b4_12_grad_x", "all_base_p8_12_split_grad_alpha", "final_accumulate_b4_12_traceable",
                 "final_accumulate_p8_12_grad_dz_ptr", "final_accumulate_b4_8_grad_beta_ptr",
                 "triangular_accumulate_b4_12_ptr_active11", "triangular_accumulate_b4_8_ptr_active7_grad_fused",
                 "triangular_accumulate_b4_12_ptr_active3_grad_gamma", "cell_mean_b4_traceable",
                 "cell_mean_b4_backward_traceable"):
        assert hasattr(torch.ops.sihc, name), name
    schema = str(torch.ops.sihc.final_accumulate_b4_12_traceable.default._schema)
    assert "Tensor dz11" in schema and "Tensor beta11" in schema
    with pytest.raises(ValueError, match=r"active must be in \[1, 11\]"):
        LK._make_triangular(12, 12)
    with pytest.raises(ValueError, match=r"all_base_b4_12_split expects x0 \[B,64,64,C\] and alpha \[12,C,16\]"):
        LK.all_base_b4_12_split_traceable(torch.randn(1, 32, 32, 8), torch.randn(12, 8, 16))
    with pytest.raises(ValueError, match=r"all_base_p8_12_split expects x0 \[B,32,32,C\] and alpha \[12,C,4\]"):
        LK.all_base_p8_12_split_traceable(torch.randn(1, 32, 32, 8), torch.randn(8, 8, 4))
    with pytest.raises(ValueError, match="CUDA device"):
        LK.all_base_b4_8_split_traceable(torch.randn(1, 64, 64, 8), torch.randn(8, 8, 16))
    with pytest.raises(ValueError, match=r"final_accumulate_p8_12 expects x0 \[B,32,32,C\]"):
        LK.final_accumulate_p8_12_traceable(torch.randn(1, 64, 64, 8), *[torch.randn(1, 256, 8)] * 12,
                                            *[torch.randn(8, 4)] * 12)
    with pytest.raises(ValueError, match="beta3 must be"):
        betas = [torch.randn(8, 16)] * 8
        betas[3] = torch.randn(8, 4)
        LK.final_accumulate_b4_8_traceable(torch.randn(1, 64, 64, 8), *[torch.randn(1, 256, 8)] * 8, *betas)
    base = torch.randn(1, 256, 8)
    ops = LK.triangular_accumulate_b4_12_ptr_active_traceable_ops
    with pytest.raises(ValueError, match=r"expects base \[B,256,C\] and gamma \[12,C\]"):
        ops[0](base, *[base] * 12, torch.randn(11, 8))
    with pytest.raises(ValueError, match="dz4 shape"):
        dzs = [base] * 12
        dzs[4] = torch.randn(1, 255, 8)
        ops[2](base, *dzs, torch.randn(12, 8))
    with pytest.raises(ValueError, match=r"cell_mean_b4 expects x \[B,64,64,C\]"):
        LK.cell_mean_b4_traceable(torch.randn(1, 32, 32, 8))

"""The split planner (tableSplit.ts:125-287): the oracle and the C ABI against the known answers
quoted in the reference's own text, and against each other on a sweep of limits."""
import numpy as np
import pytest

ROWS, ROW_BYTES = 262144, 4480  # the PLE table (tableSplit.ts:10-12)
GIB = 1 << 30


def test_known_answer_one_gib_limit(oracle, g4):
    # tableSplit.ts:68-77: a 1,073,694,720-byte first slice at a 1 GiB limit.
    o = oracle.plan_table_split(ROWS, ROW_BYTES, GIB, GIB, GIB)
    assert o["slices"][0][1] * ROW_BYTES == 1_073_694_720
    assert o["slices"] == [(0, 239664), (239664, 22480)]
    plan, slices = g4.plan_table_split(ROWS, ROW_BYTES, GIB, GIB, 10, GIB)
    assert [(s.start_row, s.row_count) for s in slices] == o["slices"]
    assert slices[0].byte_length == 1_073_694_720 and slices[1].byte_offset == 1_073_694_720
    assert plan.num_slices == 2 and not plan.single and plan.feasible
    assert plan.storage_bindings_per_dispatch == 4 and plan.dispatches_per_gather == 2


def test_known_answer_default_cap_five_slices(oracle, g4):
    o = oracle.plan_table_split(ROWS, ROW_BYTES, GIB, GIB)  # DEFAULT_MAX_SLICE_BYTES = 256 MiB
    assert o["slices"] == [(0, 59904), (59904, 59904), (119808, 59904), (179712, 59904),
                           (239616, 22528)]
    plan, slices = g4.plan_table_split(ROWS, ROW_BYTES, GIB, GIB, 10, 0)
    assert [(s.start_row, s.row_count) for s in slices] == o["slices"]


def test_known_answer_spec_floor_nine_slices(oracle, g4):
    # tableSplit.ts:26 and embedGather.ts:536-540: nine slices at the 128 MiB floor.
    floor = 134_217_728
    o = oracle.plan_table_split(ROWS, ROW_BYTES, floor, floor)
    assert len(o["slices"]) == 9
    plan, slices = g4.plan_table_split(ROWS, ROW_BYTES, floor, floor, 10, 0)
    assert plan.num_slices == 9
    assert all(s.start_row % 16 == 0 for s in slices)


def test_known_answer_m1_single_buffer(oracle, g4):
    # tableSplit.ts:13-16: the M1 grants 4,294,967,292, so the table is one binding.
    lim = 4_294_967_292
    o = oracle.plan_table_split(ROWS, ROW_BYTES, lim, lim)
    assert o["slices"] == [(0, ROWS)]
    plan, slices = g4.plan_table_split(ROWS, ROW_BYTES, lim, lim, 10, 0)
    assert plan.single and plan.num_slices == 1 and plan.rows_per_slice == ROWS


def test_infeasible_and_binding_budget(g4):
    plan, slices = g4.plan_table_split(ROWS, ROW_BYTES, 1000, 1000, 10, 0)
    assert plan.num_slices == 0 and not plan.feasible and plan.rows_per_slice == 0
    plan, slices = g4.plan_table_split(ROWS, ROW_BYTES, GIB, GIB, 3, 0)
    assert plan.num_slices == 5 and not plan.feasible  # 4 bindings do not fit a budget of 3


def test_slice_for_row(g4):
    plan, slices = g4.plan_table_split(ROWS, ROW_BYTES, GIB, GIB, 10, 0)
    assert g4.slice_for_row(slices, 0) == 0
    assert g4.slice_for_row(slices, 59903) == 0 and g4.slice_for_row(slices, 59904) == 1
    assert g4.slice_for_row(slices, ROWS - 1) == 4 and g4.slice_for_row(slices, ROWS) == -1


@pytest.mark.parametrize("limit", [1 << 20, 5_000_000, 77_777_777, 200_000_000, 600_000_000])
@pytest.mark.parametrize("cap", [0, 1 << 24, 1 << 28, 1 << 31])
def test_oracle_and_abi_agree_on_sweep(oracle, g4, limit, cap):
    o = oracle.plan_table_split(ROWS, ROW_BYTES, limit, limit * 2, cap if cap else 256 << 20)
    plan, slices = g4.plan_table_split(ROWS, ROW_BYTES, limit, limit * 2, 10, cap)
    assert [(s.start_row, s.row_count) for s in slices] == o["slices"]
    total = sum(c for _, c in o["slices"])
    assert total == ROWS  # the slices partition the vocabulary


def test_plan_gather_split_ple_at_spec_floor(oracle, g4):
    """planGatherSplit (tableSplit.ts:257-287): at the 128 MiB floor the PLE codes take nine slices
    and the scales, 262144 x 35 f32 = 36,700,160 bytes (the figure tableSplit.ts:249-255 states),
    stay one buffer, which is what the sliced gather assumes."""
    floor = 134_217_728
    plans, cs, ss = g4.plan_gather_split(ROWS, ROW_BYTES, 35, floor, floor)
    assert plans.codes.num_slices == 9 and not plans.codes.single
    assert plans.scales.total_bytes == 36_700_160
    assert plans.scales.single and plans.scales_single == 1 and len(ss) == 1
    assert [(s.start_row, s.row_count) for s in cs] == oracle.plan_table_split(
        ROWS, ROW_BYTES, floor, floor)["slices"]


def test_plan_gather_split_scales_not_single(oracle, g4):
    """Below 36.7 MB per binding the scale table itself splits: scalesSingle is false, the plan the
    gather kernel does not implement (tableSplit.ts:276-283)."""
    lim = 16 << 20
    plans, cs, ss = g4.plan_gather_split(ROWS, ROW_BYTES, 35, lim, lim)
    assert plans.scales_single == 0 and plans.scales.num_slices == len(ss) == 3
    assert [(s.start_row, s.row_count) for s in ss] == oracle.plan_table_split(
        ROWS, 35 * 4, lim, lim)["slices"]
    assert [(s.start_row, s.row_count) for s in cs] == oracle.plan_table_split(
        ROWS, ROW_BYTES, lim, lim)["slices"]


@pytest.mark.parametrize("limit", [8 << 20, 100_000_000, 1 << 30, 4_294_967_292])
def test_plan_gather_split_is_two_table_plans(oracle, g4, limit):
    plans, cs, ss = g4.plan_gather_split(ROWS, ROW_BYTES, 35, limit, limit, 10)
    for plan, slices, row_bytes in ((plans.codes, cs, ROW_BYTES), (plans.scales, ss, 140)):
        o = oracle.plan_table_split(ROWS, row_bytes, limit, limit)
        assert [(s.start_row, s.row_count) for s in slices] == o["slices"]
        assert plan.feasible == 1
    assert plans.scales_single == plans.scales.single

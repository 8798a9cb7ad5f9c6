"""Pins of the oracle's embedGather restatement (CPU) against a numpy gather + dequant."""
import numpy as np
import pytest

import npref


def numpy_gather(codes, scales, ids, cols, group):
    c = npref.codes_int4(codes[ids])                               # [T, cols]
    s = scales.astype(np.float32)[ids]                             # [T, groups]
    scale = (np.float32(16.0) * np.repeat(s, group, axis=1)).astype(np.float32)
    return (c.astype(np.float32) * scale).astype(np.float32)


@pytest.mark.parametrize("scale_dtype", [np.float32, np.float16])
@pytest.mark.parametrize("group", [256, 8960])
def test_gather_matches_numpy(oracle, scale_dtype, group):
    g = np.random.default_rng(21)
    rows, cols = 300, 8960
    codes = g.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    scales = g.uniform(0.005, 0.02, size=(rows, cols // group)).astype(scale_dtype)
    ids = g.integers(0, rows, size=37).astype(np.int32)
    want = numpy_gather(codes, scales, ids, cols, group)
    got32 = oracle.embed_gather(codes, scales, ids, cols, group, "f32")
    assert np.array_equal(got32.view(np.uint32), want.view(np.uint32))
    got16 = oracle.embed_gather(codes, scales, ids, cols, group, "f16")
    assert np.array_equal(got16.view(np.uint16), want.astype(np.float16).view(np.uint16))
    codes_out = oracle.embed_gather(codes, scales, ids, cols, group, "i8")
    assert np.array_equal(codes_out, npref.codes_int4(codes[ids]).astype(np.int8))


def test_sliced_gather_writes_only_its_slots(oracle):
    g = np.random.default_rng(22)
    rows, cols = 200, 512
    codes = g.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    scales = g.uniform(0.005, 0.02, size=(rows, 2)).astype(np.float16)
    ids = g.integers(0, rows, size=50).astype(np.int32)
    full = oracle.embed_gather(codes, scales, ids, cols, 256, "f32")
    out = np.full((ids.size, cols), -7.0, np.float32)  # sentinel: unwritten slots keep it
    for start, count in ((0, 64), (64, 64), (128, 72)):
        oracle.embed_gather(codes[start:start + count], scales, ids, cols, 256, "f32", sliced=True,
                            slice_start=start, slice_count=count, out=out)
        inside = (ids >= start) & (ids < start + count)
        assert np.array_equal(out[inside], full[inside])
    assert np.array_equal(out, full)
    part = np.full((ids.size, cols), -7.0, np.float32)
    oracle.embed_gather(codes[64:128], scales, ids, cols, 256, "f32", sliced=True, slice_start=64,
                        slice_count=64, out=part)
    outside = (ids < 64) | (ids >= 128)
    assert np.all(part[outside] == -7.0)

"""GPU parity of the PLE gather (ple-gather-4bit, -sliced, and the fused split gather).

Config 3 at full size: the int4 table of 262144 rows x 8960 columns (1,174,405,120 bytes of codes)
with f16 scales, split into 2 and into 5 vocabulary slices by the planner, Zipf(1.1) ids for 1, 64
and 2048 tokens, f16 output. Codes and f16 outputs are compared bit for bit with the oracle.
"""
import numpy as np
import pytest

import g4synth as syn

pytestmark = pytest.mark.gpu

GIB = 1 << 30


def dev(g4, a):
    return g4.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_buf(g4, shape, dtype):
    b = g4.DeviceBuffer.empty(shape, dtype)
    b.fill(0x7B)
    return b


@pytest.mark.parametrize("scale_dtype", [np.float16, np.float32])
@pytest.mark.parametrize("out_kind", ["f16", "f32", "i8"])
def test_small_table_unsliced(gpu, oracle, scale_dtype, out_kind):
    rows, cols = 5000, 8960
    g = np.random.default_rng(61)
    codes = g.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    scales = g.uniform(0.005, 0.02, size=(rows, 35)).astype(scale_dtype)
    ids = g.integers(0, rows, size=77).astype(np.int32)
    ids[:3] = [0, rows - 1, 17]
    dt = {"f16": np.float16, "f32": np.float32, "i8": np.int8}[out_kind]
    print(f"gather small scales={np.dtype(scale_dtype)} out={out_kind}", flush=True)
    out = out_buf(gpu, (ids.size, cols), dt)
    gpu.bind("ple-gather-4bit", {"codes": dev(gpu, codes), "scales": dev(gpu, scales),
                                 "ids": dev(gpu, ids)}, out, {"slots": ids.size})
    want = oracle.embed_gather(codes, scales, ids, cols, 256, out_kind)
    assert np.array_equal(out.download().view(np.uint8), want.view(np.uint8))


def test_per_row_scale_variant_and_out_of_table_ids(gpu, oracle):
    # The literal per-row variant (groupSize 8960, one scale per row), and ids past the table,
    # which the unsliced gather writes as zeros.
    rows, cols = 300, 8960
    g = np.random.default_rng(62)
    codes = g.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    scales = g.uniform(0.005, 0.02, size=(rows, 1)).astype(np.float16)
    ids = np.array([5, 299, 300, 7, 1 << 30], np.int32)
    out = out_buf(gpu, (ids.size, cols), np.float16)
    gpu.ple_gather(dev(gpu, codes), dev(gpu, scales), dev(gpu, ids), out, ids.size, cols, 8960,
                   False, 0, rows)
    got = out.download()
    ok = ids < rows
    want = oracle.embed_gather(codes, scales, ids[ok], cols, 8960, "f16")
    assert np.array_equal(got[ok].view(np.uint16), want.view(np.uint16))
    assert np.all(got[~ok].view(np.uint16) == 0)


@pytest.fixture(scope="module")
def table(gpu):
    rows, cols = syn.PLE_ROWS, syn.PLE_COLS
    print("building the 1.17 GB PLE table", flush=True)
    codes = syn.ple_codes("c3", rows)
    scales = syn.ple_scales("c3", rows)
    return codes, scales, dev(gpu, scales)


@pytest.mark.parametrize("slices_wanted", [2, 5])
@pytest.mark.parametrize("tokens", [1, 64, 2048])
def test_config3_split_table(gpu, oracle, table, slices_wanted, tokens):
    codes, scales, sb = table
    rows, cols = syn.PLE_ROWS, syn.PLE_COLS
    cap = GIB if slices_wanted == 2 else 0  # 1 GiB slices -> 2; the 256 MiB default -> 5
    plan, slices = gpu.plan_table_split(rows, cols // 2, GIB, GIB, 10, cap)
    assert plan.num_slices == slices_wanted
    ids = syn.zipf_ids("c3", tokens)
    starts = [s.start_row for s in slices]
    nb = min(tokens, len(starts))
    ids[:nb] = starts[:nb]  # slice boundaries
    print(f"config3 slices={slices_wanted} tokens={tokens}", flush=True)
    bufs = [dev(gpu, codes[s.start_row:s.start_row + s.row_count]) for s in slices]
    idb = dev(gpu, ids)
    want = oracle.embed_gather(codes, scales, ids, cols, 256, "f16")
    # One dispatch per slice, as the reference walks slicedGatherDispatches.
    out = out_buf(gpu, (tokens, cols), np.float16)
    for s, b in zip(slices, bufs):
        gpu.bind("ple-gather-4bit-sliced", {"codes": b, "scales": sb, "ids": idb}, out,
                 {"slots": tokens, "sliceStartRow": s.start_row, "sliceRowCount": s.row_count})
    assert np.array_equal(out.download().view(np.uint16), want.view(np.uint16))
    # The fused launch over every slice.
    out2 = out_buf(gpu, (tokens, cols), np.float16)
    gpu.ple_gather_split(bufs, [s.start_row for s in slices], [s.row_count for s in slices], sb,
                         idb, out2, tokens, cols, 256)
    assert np.array_equal(out2.download().view(np.uint16), want.view(np.uint16))
    # Gathered codes, bit for bit.
    oc = out_buf(gpu, (tokens, cols), np.int8)
    gpu.ple_gather_split(bufs, [s.start_row for s in slices], [s.row_count for s in slices], sb,
                         idb, oc, tokens, cols, 256)
    assert np.array_equal(oc.download(), oracle.embed_gather(codes, scales, ids, cols, 256, "i8"))
    for b in bufs:
        b.close()


def test_sliced_dispatch_leaves_other_slots(gpu, oracle, table):
    codes, scales, sb = table
    cols = syn.PLE_COLS
    plan, slices = gpu.plan_table_split(syn.PLE_ROWS, cols // 2, GIB, GIB, 10, 0)
    s = slices[1]
    ids = np.array([s.start_row - 1, s.start_row, s.start_row + s.row_count - 1,
                    s.start_row + s.row_count, 3], np.int32)
    out = out_buf(gpu, (ids.size, cols), np.float16)
    b = dev(gpu, codes[s.start_row:s.start_row + s.row_count])
    gpu.ple_gather(b, sb, dev(gpu, ids), out, ids.size, cols, 256, True, s.start_row, s.row_count)
    got = out.download().view(np.uint16)
    inside = np.array([False, True, True, False, False])
    want = oracle.embed_gather(codes, scales, ids[inside], cols, 256, "f16")
    assert np.array_equal(got[inside], want.view(np.uint16))
    assert np.all(got[~inside] == 0x7B7B)  # untouched: still the sentinel

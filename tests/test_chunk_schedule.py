"""CPU: the chunk schedule of the chunk driver and the driver's host-side preflight.

The schedule cases restate the reference's tests/metal/prefill_chunk_test.cpp:129-260
(builds_chunk_schedule_without_padding, rejects_invalid_chunk_schedules_transactionally):
ranges are contiguous, unpadded, keep absolute positions and cover every token once; bad
chunk sizes and positions past the signed StepRow range are rejected with the output left
unchanged; an out-of-range lookup leaves its output unchanged.
"""
import ctypes as C

import pytest

from test_abi_host import Fake

INT32_MAX = 2 ** 31 - 1
MAX_ROWS = 419430


@pytest.fixture
def fake(moe):
    return Fake(moe)


def test_schedule_without_padding(moe):
    sched, err = moe.build_chunk_schedule(7, 10, 4)
    assert sched is not None, err
    assert (sched.token_count, sched.chunk_rows) == (10, 4)
    assert moe.chunk_ranges(sched) == [(0, 7, 4), (4, 11, 4), (8, 15, 2)]
    assert sum(r[2] for r in moe.chunk_ranges(sched)) == 10
    lib = moe.library()
    untouched = moe.ChunkRange(91, 92, 93)
    assert lib.sm_chunk_range_at(C.byref(sched), 3, C.byref(untouched)) == 0
    assert (untouched.token_offset, untouched.pos0, untouched.rows) == (91, 92, 93)
    empty, err = moe.build_chunk_schedule(2 ** 32 - 1, 0, 4)
    assert empty is not None and moe.chunk_ranges(empty) == [] and empty.chunk_rows == 4


def test_schedule_rejections_leave_output_unchanged(moe):
    lib = moe.library()
    sched, _ = moe.build_chunk_schedule(17, 3, 3)
    err = C.create_string_buffer(256)

    def build(pos0, n, rows):
        return lib.sm_build_chunk_schedule(pos0, n, rows, C.byref(sched), err, 256)

    def unchanged(pos0, n, rows):
        return (sched.pos0, sched.token_count, sched.chunk_rows) == (pos0, n, rows)

    assert build(0, 3, 0) != 0 and b"shader row limit" in err.value and unchanged(17, 3, 3)
    assert build(0, 3, MAX_ROWS + 1) != 0 and b"shader row limit" in err.value and unchanged(17, 3, 3)
    last = INT32_MAX - 1
    assert build(last, 1, 1) == 0 and moe.chunk_ranges(sched) == [(0, last, 1)]
    assert build(last, 2, 1) != 0 and b"signed StepRow" in err.value and unchanged(last, 1, 1)
    assert build(1, 2 ** 64 - 1, 1) != 0 and b"signed StepRow" in err.value and unchanged(last, 1, 1)


@pytest.mark.parametrize("n,rows", [(1, 1), (4096, 4096), (16384, 4096), (16385, 4096), (5, 7)])
def test_schedule_covers_every_token_once(moe, n, rows):
    sched, err = moe.build_chunk_schedule(100, n, rows)
    assert sched is not None, err
    rs = moe.chunk_ranges(sched)
    assert len(rs) == -(-n // rows)
    offs = 0
    for off, pos0, r in rs:
        assert off == offs and pos0 == 100 + off and 0 < r <= rows
        offs += r
    assert offs == n


def _driver(moe, fake, n_tokens, chunk_rows=None, **over):
    """Encodes the chunk driver over a prompt of n_tokens with fake's layer as chunk scratch."""
    chunk_rows = chunk_rows or fake.shape.rows
    d = fake.shape.hidden
    x_all, out_all = fake.buf(n_tokens * d * 2), fake.buf(n_tokens * d * 4)
    sched, err = moe.build_chunk_schedule(0, n_tokens, chunk_rows)
    assert sched is not None, err
    seg = fake.ctx.segment()
    ok, err = seg.encode_prefill_moe_chunks(sched, over.pop("shape", fake.shape), fake.fmts,
                                            over.pop("input", x_all.view()), over.pop("output", out_all.view()),
                                            fake.layer())
    n = seg.launches
    seg.abort()
    return ok, err, n


def test_driver_encodes_every_chunk(moe, fake):
    ok, err, n = _driver(moe, fake, 3 * fake.shape.rows + 2)
    assert ok, err
    assert n == 4 * 10  # four chunks (the last of 2 rows), 10 launches each


def test_driver_rejections(moe, fake):
    # scratch rows must be the schedule's chunk size
    ok, err, _ = _driver(moe, fake, 20, chunk_rows=fake.shape.rows - 1)
    assert not ok and "scratch rows must equal" in err
    # an input view too short for the prompt
    short = fake.buf(16)
    ok, err, _ = _driver(moe, fake, 20, input=short.view())
    assert not ok and "input rows view is undersized" in err
    # output on top of the input
    x = fake.buf(20 * fake.shape.hidden * 4)
    ok, err, _ = _driver(moe, fake, 20, input=x.view(0, 20 * fake.shape.hidden * 2), output=x.view())
    assert not ok and "output rows overlaps active input rows" in err
    # a chunk's output slice on top of chunk scratch (the gathered rows)
    ok, err, _ = _driver(moe, fake, fake.shape.rows, output=fake.xs.view(0, fake.shape.rows * fake.shape.hidden * 4))
    assert not ok and "overlaps active" in err


def test_layer_selection_in_address_table(moe, fake):
    """Two layers of one [layer][E][3] table and one plans buffer, in one segment."""
    E = fake.shape.n_experts
    table = list(fake.addr) + list(fake.addr)
    plans = fake.buf(2 * 6400)
    seg = fake.ctx.segment()
    for layer in (0, 1):
        lb = fake.layer(views={"plan": plans.view(6400 * layer, 6400)})
        for st in (lb.gate_up, lb.down):
            st.weights.n_layers = 2
            st.weights.layer = layer
        keep = moe.ExpertTable(table, lb.gate_up.weights.address_snapshot, [fake.w_gate.view(), fake.w_up.view()],
                               n_layers=2, layer=layer)
        lb.gate_up.weights = keep.struct
        keep2 = moe.ExpertTable(table, lb.down.weights.address_snapshot, [fake.w_down.view()], n_layers=2, layer=layer)
        lb.down.weights = keep2.struct
        ok, err = seg.encode_prefill_moe_full_mode_layer(fake.shape, fake.fmts, lb, keep=(keep, keep2))
        assert ok, err
    assert seg.launches == 20
    seg.abort()
    lb = fake.layer()
    lb.gate_up.weights.layer = 1  # n_layers is 1
    seg = fake.ctx.segment()
    ok, err = seg.encode_prefill_moe_full_mode_layer(fake.shape, fake.fmts, lb)
    seg.abort()
    assert not ok and "layer is outside the address table" in err

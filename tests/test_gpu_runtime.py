"""Runtime pieces on the GPU: event records captured into a graph time the kernels
between them on every replay (the bench's in-step kernel timing relies on it)."""
import numpy as np
import pytest

from tabinfer_amd import abi

pytestmark = pytest.mark.gpu


def test_event_records_inside_a_graph_time_each_replay():
    with abi.Ctx(0) as ctx:
        n = 64 << 20
        a, b = ctx.zeros(n), ctx.zeros(n)
        ctx.sync()
        ctx.graph_begin()
        ctx.record(0)
        ctx.call("ti_buf_copy", b, 0, a, 0, n)
        ctx.record(1)
        ctx.call("ti_buf_fill_u32", a, 7, n // 4)
        ctx.record(2)
        g = ctx.graph_end()
        try:
            for rep in range(3):
                ctx.graph_launch(g)
                ctx.sync()
                t01, t12 = ctx.elapsed_ms(0, 1), ctx.elapsed_ms(1, 2)
                assert 0.0 < t01 < 50.0 and 0.0 < t12 < 50.0, (rep, t01, t12)
                assert int(ctx.download(a, np.uint32, 1)[0]) == 7
        finally:
            ctx.graph_destroy(g)

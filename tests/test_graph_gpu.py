"""HIP graph capture and replay of flash launches (the extension the benchmark times with).

One graph holds two launches of different shapes (causal d=64 and non-causal d=32). It is replayed
several times. Between replays the test clears the graph's outputs and issues eager launches of
another shape into other buffers, and synchronizes. Every replay must reproduce the eager outputs
bit for bit.
"""

import sys

import numpy as np
import pytest

import notcute_flash as nc
from flash_workloads import Workload

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _device(wl):
    q, k, v = wl.make_inputs()
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v)]
    o = nc.DeviceBuffer(wl.length("o") * 4)
    o.memset(0)
    return bufs + [o]


def test_graph_replays_match_eager(gpu):
    wa = Workload("graph_a", 4, 700, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=41)
    wb = Workload("graph_b", 3, 333, 32, False, 32 ** -0.5, (("normal", 0.0, 1.0),) * 3, seed=42)
    wc = Workload("graph_eager", 2, 150, 16, True, 0.25, (("uniform", -1.0, 1.0),) * 3, seed=43)
    say(f"[case] graph of {wa.describe()} + {wb.describe()}; eager {wc.describe()} between replays")
    a, b, c = _device(wa), _device(wb), _device(wc)
    stream = nc.Stream()
    graph = None
    try:
        def launch(w, bufs):
            nc.flash_launch(gpu, *bufs, w.options(), stream=stream.handle)

        launch(wa, a)
        launch(wb, b)
        stream.synchronize()
        ref_a = a[3].download(np.float32, wa.length("o"))
        ref_b = b[3].download(np.float32, wb.length("o"))

        graph = nc.Graph.capture(stream, lambda: (launch(wa, a), launch(wb, b)))
        for r in range(4):
            a[3].memset(0)
            b[3].memset(0)
            nc.synchronize()  # the clears (null stream) are done before the non-blocking stream runs
            launch(wc, c)  # eager work of another shape on the same stream
            stream.synchronize()
            graph.launch(stream)
            launch(wc, c)
            stream.synchronize()
            out_a = a[3].download(np.float32, wa.length("o"))
            out_b = b[3].download(np.float32, wb.length("o"))
            assert np.array_equal(out_a.view(np.uint32), ref_a.view(np.uint32)), f"replay {r}: graph_a differs"
            assert np.array_equal(out_b.view(np.uint32), ref_b.view(np.uint32)), f"replay {r}: graph_b differs"
            say(f"[ok] replay {r}")
    finally:
        if graph is not None:
            graph.destroy()
        stream.destroy()
        for buf in a + b + c:
            buf.free()


def test_event_record_nodes_bracket_launches_inside_a_graph(gpu):
    """nc_event_record_node during a capture puts the event records into the graph (bench.py times
    its K launches this way): every replay records both events; the pair brackets only the launches
    between them, so it measures less than an event pair recorded around the whole replay, which also
    holds the two launches before the first node and the graph's own launch; and the launches inside
    still compute the eager result."""
    wl = Workload("graph_nodes", 8, 512, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=44)
    say(f"[case] record nodes around 10 launches of {wl.describe()}")
    bufs = _device(wl)
    stream = nc.Stream()
    n0, n1 = nc.Event(timing_only=True), nc.Event(timing_only=True)
    o0, o1 = nc.Event(timing_only=True), nc.Event(timing_only=True)
    graph = None
    try:
        def launch():
            nc.flash_launch(gpu, *bufs, wl.options(), stream=stream.handle)

        launch()
        stream.synchronize()
        ref = bufs[3].download(np.float32, wl.length("o"))

        def body():
            launch()
            launch()
            n0.record_node(stream.handle)
            for _ in range(10):
                launch()
            n1.record_node(stream.handle)

        graph = nc.Graph.capture(stream, body)
        for r in range(3):
            bufs[3].memset(0)
            nc.synchronize()
            o0.record(stream.handle)
            graph.launch(stream)
            o1.record(stream.handle)
            stream.synchronize()
            inside, outside = nc.Event.elapsed(n0, n1), nc.Event.elapsed(o0, o1)
            out = bufs[3].download(np.float32, wl.length("o"))
            assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), f"replay {r}: output differs"
            assert 0.0 < inside < outside, f"replay {r}: inside {inside} ms, outside {outside} ms"
            say(f"[ok] replay {r}: 10 launches {inside * 1e3:.1f} us between the nodes, "
                f"{outside * 1e3:.1f} us around the replay")
    finally:
        if graph is not None:
            graph.destroy()
        stream.destroy()
        for e in (n0, n1, o0, o1):
            e.destroy()
        for buf in bufs:
            buf.free()

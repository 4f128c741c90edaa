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

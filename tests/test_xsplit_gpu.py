"""GPU parity of the pair-split causal kernels (nc_flash_fwd_d64_q1s8p2x_causal[_bf16]).

The query blocks p and nqb-1-p of a head are shared by two workgroups, which exchange their
partials of the heavier block through a scratch buffer and a per-pair counter that every launch
advances by two (the workgroup that finds it odd merges). The dispatch picks these kernels only for
long causal sequences over few heads (at least 96 query blocks, at most 256 workgroups), so most
cases here launch the kernel by name with a scratch buffer of their own, on shapes of every kind
(odd and even block counts, S not a multiple of 32, batch_heads not a multiple of 8, which puts the
two workgroups of a pair on different XCDs, bf16); the dispatched shapes go through nc_flash_launch
and the library's static scratch. Beyond the oracle, the tests launch repeatedly with the same and
with changing inputs, alternate shapes that share one scratch buffer (whose counters then overlap),
capture a module's first launch into a HIP graph, grow the by-name workspace under a captured graph
and replay graphs: a counter left odd or a stale partial would show as a wrong row.
"""

import numpy as np
import pytest

import flashcheck as fc
import notcute_flash as nc
from flash_workloads import Workload

pytestmark = pytest.mark.gpu

XS = "nc_flash_fwd_d64_q1s8p2x_causal"


def _wl(bh, s, seed, dtype="f16", sigma=1.0, **kw):
    wl = Workload(f"xs_bh{bh}_s{s}_{dtype}", bh, s, 64, True, 0.125, (("normal", 0.0, sigma),) * 3, seed=seed, **kw)
    wl.dtype = dtype
    return wl


SHAPES = [(1, 33), (1, 64), (2, 65), (3, 100), (1, 257), (5, 300), (8, 512), (3, 999), (8, 1024), (4, 1056),
          (2, 2048), (1, 4096)]
DISPATCHED = [(1, 3072), (1, 4096), (2, 3100), (2, 4096), (1, 8192)]


class Scratch:
    """A zeroed scratch buffer of its own for direct launches of the pair-split kernel."""

    def __init__(self, nbytes):
        self.buf = nc.DeviceBuffer(nbytes)
        self.buf.memset(0)

    def launch(self, mod, wl, bufs, stream=None):
        name = XS + ("_bf16" if wl.dtype == "bf16" else "")
        opts = wl.options()
        need = nc.kernel_scratch_bytes(name, opts)
        assert 0 < need <= self.buf.nbytes
        sel = nc.KernelSelection()
        sel.block_m = 32
        args = nc.pack_args(opts, sel, *[b.ptr for b in bufs])
        args.scratch = self.buf.ptr
        mod.get_function(name).launch((((wl.seq_len + 31) // 32) * wl.batch_heads,), (512,), [args], stream=stream)

    def free(self):
        self.buf.free()


class Run:
    """Device buffers of one workload, launched through nc_flash_launch."""

    def __init__(self, wl, q, k, v, o_init):
        self.wl = wl
        self.bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]

    def launch(self, mod, stream=None):
        nc.flash_launch(mod, *self.bufs, self.wl.options(), stream=stream)

    def output(self):
        nc.synchronize()
        return self.bufs[3].download(np.float32, self.wl.length("o"))

    def upload(self, q, k, v):
        for b, x in zip(self.bufs, (q, k, v)):
            b.upload(x)

    def free(self):
        for b in self.bufs:
            b.free()


def _check(out, ref, wl, o_init, what):
    bar_abs, bar_rel = fc.parity_bar(wl.dtype)
    ea, er = fc.assert_parity(out, ref, fc.active_index(wl), what, max_abs=bar_abs, max_rel=bar_rel)
    fc.assert_pads_untouched(out, o_init, wl, what)
    return ea, er


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("bh,s", SHAPES, ids=[f"bh{b}_s{s}" for b, s in SHAPES])
def test_pair_split_parity(gpu, bh, s, dtype):
    wl = _wl(bh, s, seed=40 + s + bh, dtype=dtype, o_stride=s * 64 + 12)
    q, k, v = wl.make_inputs()
    o_init = np.full(wl.length("o"), fc.SENTINEL, dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    print(f"[case] {wl.describe()} {dtype} direct", flush=True)
    scratch = Scratch(nc.kernel_scratch_bytes(XS, wl.options()))
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    try:
        scratch.launch(gpu, wl, bufs)
        nc.synchronize()
        out = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
        scratch.free()
    ea, er = _check(out, ref, wl, o_init, wl.name)
    print(f"[ok] max-abs {ea:.2e} max-rel {er:.2e}", flush=True)


@pytest.mark.parametrize("bh,s", DISPATCHED, ids=[f"bh{b}_s{s}" for b, s in DISPATCHED])
def test_pair_split_dispatched(gpu, bh, s):
    """Shapes the dispatch sends to the pair split, through nc_flash_launch and the static scratch."""
    wl = _wl(bh, s, seed=60 + s + bh)
    sel = nc.select_kernel(wl.options())
    print(f"[case] {wl.describe()} -> {sel.name.decode()} scratch {sel.scratch_bytes}", flush=True)
    assert sel.name.decode() == XS and sel.scratch_bytes > 0
    rows = np.unique(np.concatenate([np.arange(0, s, 37), np.arange(s - 40, s)]))
    q, k, v = wl.make_inputs()
    o_init = np.zeros(wl.length("o"), dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    out = fc.run_gpu(gpu, wl, q, k, v, o_init)
    ea, er = fc.assert_parity(out, ref, fc.active_index(wl, rows), wl.name)
    print(f"[ok] max-abs {ea:.2e} max-rel {er:.2e}", flush=True)


def test_pair_split_large_logits(gpu):
    """Q, K ~ N(0, 3) (c5's distribution) at c3's shape: the partials' maxima differ widely."""
    wl = Workload("xs_c3_sigma3", 8, 1024, 64, True, 0.125,
                  (("normal", 0.0, 3.0), ("normal", 0.0, 3.0), ("uniform", -1.0, 1.0)), seed=51)
    q, k, v = wl.make_inputs()
    o_init = np.zeros(wl.length("o"), dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, o_init=o_init)
    scratch = Scratch(nc.kernel_scratch_bytes(XS, wl.options()))
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    try:
        scratch.launch(gpu, wl, bufs)
        nc.synchronize()
        out = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
        scratch.free()
    ea, er = _check(out, ref, wl, o_init, wl.name)
    print(f"[ok] max-abs {ea:.2e} max-rel {er:.2e}", flush=True)


def test_pair_split_repeated_launches(gpu):
    """Seven launches in a row on the same buffers (each checked, and bitwise equal: the merge does
    not depend on which workgroup of a pair arrives last), then new inputs in the same buffers: every
    launch must merge the current launch's partials (dispatched shape)."""
    wl = _wl(1, 4096, seed=57)
    rows = np.arange(0, 4096, 17)
    q, k, v = wl.make_inputs()
    o_init = np.zeros(wl.length("o"), dtype=np.float32)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    idx = fc.active_index(wl, rows)
    run = Run(wl, q, k, v, o_init)
    try:
        first = None
        for i in range(7):
            run.bufs[3].memset(0)
            run.launch(gpu)
            out = run.output()
            fc.assert_parity(out, ref, idx, f"launch {i}")
            if first is None:
                first = out
            assert np.array_equal(out.view(np.uint32), first.view(np.uint32)), f"launch {i} differs from launch 0"
        wl2 = _wl(1, 4096, seed=58)
        q2, k2, v2 = wl2.make_inputs()
        ref2 = fc.oracle(wl2, q2, k2, v2, rows=rows, o_init=o_init)
        run.upload(q2, k2, v2)
        for i in range(3):
            run.launch(gpu)
            fc.assert_parity(run.output(), ref2, idx, f"new inputs, launch {i}")
    finally:
        run.free()


def test_pair_split_shapes_share_a_scratch_buffer(gpu):
    """Three shapes with different pair counts alternate on one scratch buffer (their counters
    overlap, and each shape's slots lie over the others' earlier partials); every output checked."""
    cases = [_wl(2, 300, seed=53), _wl(8, 1024, seed=54), _wl(4, 4096, seed=55)]
    scratch = Scratch(max(nc.kernel_scratch_bytes(XS, wl.options()) for wl in cases))
    bufs, refs = [], []
    try:
        for wl in cases:
            q, k, v = wl.make_inputs()
            o_init = np.zeros(wl.length("o"), dtype=np.float32)
            refs.append(fc.oracle(wl, q, k, v, o_init=o_init))
            bufs.append([nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)])
        for n, i in enumerate([0, 1, 0, 2, 1, 0, 2, 2, 1]):
            scratch.launch(gpu, cases[i], bufs[i])
            nc.synchronize()
            out = bufs[i][3].download(np.float32, cases[i].length("o"))
            _check(out, refs[i], cases[i], np.zeros(cases[i].length("o"), np.float32), f"step {n} ({cases[i].name})")
    finally:
        for bs in bufs:
            for b in bs:
                b.free()
        scratch.free()


def test_pair_split_dispatched_sizes_share_the_static_scratch(gpu):
    """Dispatched shapes in increasing and then decreasing size on a fresh module: all share the
    GPU's static scratch (their counters overlap); every output checked on sampled rows."""
    mod = nc.Module.load_embedded()
    try:
        for n, (bh, s) in enumerate([(1, 3072), (2, 4096), (1, 8192), (2, 3100), (1, 8192)]):
            wl = _wl(bh, s, seed=70 + n)
            rows = np.arange(0, s, 53)
            q, k, v = wl.make_inputs()
            o_init = np.zeros(wl.length("o"), dtype=np.float32)
            ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
            fc.assert_parity(fc.run_gpu(mod, wl, q, k, v, o_init), ref, fc.active_index(wl, rows), f"step {n}")
    finally:
        mod.unload()


def test_pair_split_graph_replays(gpu):
    """A HIP graph of three launches replayed five times, with eager launches and synchronisation
    between the replays; each replay's output equals the eager one bitwise."""
    wl = _wl(2, 4096, seed=56)
    q, k, v = wl.make_inputs()
    o_init = np.zeros(wl.length("o"), dtype=np.float32)
    run = Run(wl, q, k, v, o_init)
    stream = nc.Stream()
    try:
        run.launch(gpu, stream.handle)
        stream.synchronize()
        eager = run.output()
        rows = np.arange(0, wl.seq_len, 41)
        fc.assert_parity(eager, fc.oracle(wl, q, k, v, rows=rows, o_init=o_init), fc.active_index(wl, rows), "eager")
        graph = nc.Graph.capture(stream, lambda: [run.launch(gpu, stream.handle) for _ in range(3)])
        try:
            for i in range(5):
                run.bufs[3].memset(0)
                graph.launch(stream)
                stream.synchronize()
                out = run.output()
                assert np.array_equal(out.view(np.uint32), eager.view(np.uint32)), f"replay {i}"
                run.launch(gpu, stream.handle)  # eager work between replays
                stream.synchronize()
        finally:
            graph.destroy()
    finally:
        run.free()
        stream.destroy()


def test_first_launch_captured_into_a_graph(gpu):
    """The first nc_flash_launch of a freshly loaded module, of a pair-split shape (BH=1 S=4096
    causal) and with nothing reserved, captured into a HIP graph: the launch neither allocates nor
    synchronises, so the capture succeeds; three replays, with eager launches and synchronisation
    between them, each match the oracle and one another bitwise."""
    wl = _wl(1, 4096, seed=61)
    assert nc.select_kernel(wl.options()).name.decode() == XS
    q, k, v = wl.make_inputs()
    o_init = np.zeros(wl.length("o"), dtype=np.float32)
    rows = np.unique(np.concatenate([np.arange(0, wl.seq_len, 29), np.arange(wl.seq_len - 33, wl.seq_len)]))
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    idx = fc.active_index(wl, rows)
    mod = nc.Module.load_embedded()
    run = Run(wl, q, k, v, o_init)
    stream = nc.Stream()
    try:
        print(f"[case] {wl.describe()} first launch of a fresh module under capture", flush=True)
        graph = nc.Graph.capture(stream, lambda: run.launch(mod, stream.handle))
        try:
            first = None
            for i in range(3):
                run.bufs[3].memset(0)
                graph.launch(stream)
                stream.synchronize()
                out = run.output()
                fc.assert_parity(out, ref, idx, f"replay {i}")
                if first is None:
                    first = out
                assert np.array_equal(out.view(np.uint32), first.view(np.uint32)), f"replay {i} differs"
                run.launch(mod, stream.handle)  # eager work between replays
                stream.synchronize()
        finally:
            graph.destroy()
    finally:
        run.free()
        stream.destroy()
        mod.unload()


_FIRST_LAUNCH_PROGRAM = r"""
import sys
import numpy as np
import flashcheck as fc
import notcute_flash as nc
from flash_workloads import Workload
nc.load_library()
nc.init()
mod = nc.Module.load_embedded()
wl = Workload("xs_first", 1, 4096, 64, True, 0.125, (("normal", 0.0, 1.0),) * 3, seed=65)
assert nc.select_kernel(wl.options()).name.decode() == "nc_flash_fwd_d64_q1s8p2x_causal"
q, k, v = wl.make_inputs()
o_init = np.zeros(wl.length("o"), dtype=np.float32)
rows = np.arange(0, wl.seq_len, 37)
ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
stream = nc.Stream()
graph = nc.Graph.capture(stream, lambda: nc.flash_launch(mod, *bufs, wl.options(), stream=stream.handle))
for i in range(3):
    bufs[3].memset(0)
    graph.launch(stream)
    stream.synchronize()
    fc.assert_parity(bufs[3].download(np.float32, wl.length("o")), ref, fc.active_index(wl, rows), f"replay {i}")
graph.destroy()
print("first-launch capture ok", flush=True)
"""


def test_first_launch_of_a_process_captured(gpu):
    """In a fresh process, the very first flash launch (a pair-split shape, BH=1 S=4096 causal, no
    reserve, no eager launch before it) is captured into a HIP graph and replayed three times,
    each replay checked against the oracle."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join(os.path.join(root, d) for d in ("not-cute-zig_amd", "oracle", "tests"))
    print("[case] first launch of a fresh process, captured (subprocess)", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_LAUNCH_PROGRAM], env=env, capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "first-launch capture ok" in r.stdout


def test_by_name_workspace_outlives_growth(gpu):
    """A by-name launch captured into a graph with the workspace reserved for a small shape keeps
    working after a larger reserve on the same module grows the workspace (the old one is kept until
    the module is unloaded): replays after the growth, and after eager launches of the larger shape
    on the new workspace, match the oracle."""
    small, large = _wl(1, 3072, seed=62), _wl(1, 8192, seed=63)
    mod = nc.Module.load_embedded()
    stream = nc.Stream()
    data = {}
    try:
        for wl in (small, large):
            q, k, v = wl.make_inputs()
            o_init = np.zeros(wl.length("o"), dtype=np.float32)
            rows = np.arange(0, wl.seq_len, 47)
            data[wl.name] = (Run(wl, q, k, v, o_init), fc.oracle(wl, q, k, v, rows=rows, o_init=o_init),
                             fc.active_index(wl, rows))

        def by_name(wl, ws):
            run = data[wl.name][0]
            sel = nc.KernelSelection()
            sel.block_m = 32
            args = nc.pack_args(wl.options(), sel, *[b.ptr for b in run.bufs])
            args.scratch = ws
            mod.get_function(XS).launch((((wl.seq_len + 31) // 32) * wl.batch_heads,), (512,), [args],
                                        stream=stream.handle)

        ws_small = nc.reserve_workspace(mod, small.options())
        assert ws_small
        graph = nc.Graph.capture(stream, lambda: by_name(small, ws_small))
        try:
            ws_large = nc.reserve_workspace(mod, large.options())
            assert ws_large and ws_large != ws_small
            assert nc.reserve_workspace(mod, small.options()) == ws_large  # the larger one serves both now
            for i in range(3):
                run, ref, idx = data[small.name]
                run.bufs[3].memset(0)
                graph.launch(stream)
                stream.synchronize()
                fc.assert_parity(run.output(), ref, idx, f"small replay {i}")
                run, ref, idx = data[large.name]
                run.bufs[3].memset(0)
                by_name(large, ws_large)
                stream.synchronize()
                fc.assert_parity(run.output(), ref, idx, f"large eager {i}")
        finally:
            graph.destroy()
    finally:
        for run, _, _ in data.values():
            run.free()
        stream.destroy()
        mod.unload()


def test_reset_scratch_restores_the_counters(gpu):
    """nc_flash_reset_scratch zeroes the exchange counters: launches before and after it agree with
    the oracle (the counters are even between launches, so a reset between launches changes
    nothing a later launch sees)."""
    wl = _wl(2, 4096, seed=64)
    q, k, v = wl.make_inputs()
    o_init = np.zeros(wl.length("o"), dtype=np.float32)
    rows = np.arange(0, wl.seq_len, 31)
    ref = fc.oracle(wl, q, k, v, rows=rows, o_init=o_init)
    idx = fc.active_index(wl, rows)
    run = Run(wl, q, k, v, o_init)
    try:
        for i in range(2):
            run.launch(gpu)
            fc.assert_parity(run.output(), ref, idx, f"before reset, launch {i}")
        nc.reset_scratch(gpu)
        nc.reset_scratch()
        for i in range(2):
            run.bufs[3].memset(0)
            run.launch(gpu)
            fc.assert_parity(run.output(), ref, idx, f"after reset, launch {i}")
    finally:
        run.free()


def test_pair_split_matches_unsplit_kernel(gpu):
    """The pair-split and the plain private-staging kernel agree within the parity bar on a
    dispatched shape (the plain kernel launched by name with its own geometry)."""
    wl = _wl(1, 8192, seed=59)
    assert nc.select_kernel(wl.options()).name.decode() == XS
    q, k, v = wl.make_inputs()
    o_init = np.zeros(wl.length("o"), dtype=np.float32)
    out_x = fc.run_gpu(gpu, wl, q, k, v, o_init)
    bufs = [nc.DeviceBuffer.from_array(x) for x in (q, k, v, o_init)]
    try:
        sel = nc.KernelSelection()
        sel.block_m = 32
        args = nc.pack_args(wl.options(), sel, *[b.ptr for b in bufs])
        gpu.get_function("nc_flash_fwd_d64_q1s8p2_causal").launch((256 * wl.batch_heads,), (512,), [args])
        nc.synchronize()
        out_p = bufs[3].download(np.float32, wl.length("o"))
    finally:
        for b in bufs:
            b.free()
    idx = fc.active_index(wl)
    assert float(np.max(np.abs(out_x[idx] - out_p[idx]))) <= fc.MAX_ABS

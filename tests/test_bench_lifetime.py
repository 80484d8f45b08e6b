"""bench.py's set-up / measurement / teardown sequence against a recording fake of the HIP
layer and of libfriday_attn (CPU only, nothing runs on a GPU).

The fake hands out device addresses, records which pointers every launch issued under
stream capture passes, and fails the test when a buffer is freed while an instantiated
graph that captured a launch on it still exists: freed memory that a live graph points at
is reused by the next allocation, and a replay (or the runtime's own bookkeeping) then
touches memory that belongs to someone else."""
import ctypes as C
import os
import sys
import types

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "friday-inference-engine_amd"))
sys.path.insert(0, ROOT)


class FakeHip:
    """Recording stand-in for the libamdhip64 entry points friday_attn.Hip binds."""

    def __init__(self):
        self.next_addr = 0x7F0000000000
        self.allocs = {}          # ptr -> bytes
        self.capturing = {}       # stream -> list of pointers used by launches captured on it
        self.graphs = {}          # graph handle -> pointers
        self.execs = {}           # exec handle -> pointers (live executable graphs)
        self.streams, self.events = set(), set()
        self.handle = 1
        self.violations = []

    def _new_handle(self):
        self.handle += 1
        return self.handle

    # -- memory
    def hipMalloc(self, ref, n):
        ptr = self.next_addr
        self.next_addr += (int(n) + (1 << 20)) & ~((1 << 20) - 1)  # 1 MiB apart at least
        self.allocs[ptr] = int(n)
        ref._obj.value = ptr
        return 0

    def hipFree(self, ptr):
        n = self.allocs.pop(ptr, None)
        if n is None:
            self.violations.append(f"free of unknown pointer {ptr:#x}")
            return 1
        for e, ptrs in self.execs.items():
            if any(ptr <= p < ptr + n for p in ptrs):
                self.violations.append(f"free of {ptr:#x} ({n} B) while live graph exec {e} references it")
        return 0

    def hipMemcpy(self, dst, src, n, kind):
        return 0

    def hipMemcpyAsync(self, dst, src, n, kind, stream):
        return 0

    def hipMemset(self, p, v, n):
        return 0

    # -- streams and events
    def hipStreamCreate(self, ref):
        h = self._new_handle()
        self.streams.add(h)
        ref._obj.value = h
        return 0

    def hipStreamDestroy(self, s):
        self.streams.discard(s)
        return 0

    def hipStreamSynchronize(self, s):
        return 0

    def hipDeviceSynchronize(self):
        return 0

    def hipGetDeviceCount(self, ref):
        ref._obj.value = 1
        return 0

    def hipEventCreate(self, ref):
        h = self._new_handle()
        self.events.add(h)
        ref._obj.value = h
        return 0

    def hipEventDestroy(self, e):
        self.events.discard(e)
        return 0

    def hipEventRecord(self, e, s):
        return 0

    def hipEventSynchronize(self, e):
        return 0

    def hipEventElapsedTime(self, ref, a, b):
        ref._obj.value = 1.0
        return 0

    def hipGetErrorString(self, rc):
        return b"fake error"

    # -- graphs
    def hipStreamBeginCapture(self, s, mode):
        self.capturing[s] = []
        return 0

    def hipStreamEndCapture(self, s, ref):
        g = self._new_handle()
        self.graphs[g] = self.capturing.pop(s)
        ref._obj.value = g
        return 0

    def hipGraphInstantiate(self, ref, g, a, b, c):
        e = self._new_handle()
        self.execs[e] = list(self.graphs[g])
        ref._obj.value = e
        return 0

    def hipGraphLaunch(self, e, s):
        if e not in self.execs:
            self.violations.append(f"launch of destroyed graph exec {e}")
        return 0

    def hipGraphExecDestroy(self, e):
        self.execs.pop(e, None)
        return 0

    def hipGraphDestroy(self, g):
        self.graphs.pop(g, None)
        return 0

    # -- launches: any pointer argument inside a live allocation is recorded for the
    # captures in progress (bench issues every launch on its one stream)
    def record_launch(self, args):
        ptrs = [a for a in args if isinstance(a, int) and any(p <= a < p + n for p, n in self.allocs.items())]
        for lst in self.capturing.values():
            lst.extend(ptrs)


class FakeLib:
    """libfriday_attn stand-in: size queries return plausible sizes, launches record their pointers."""

    SIZES = {"friday_attn_rope_table_bytes": lambda mc, d: mc * d * 4,
             "friday_attn_split_workspace_bytes": lambda hq, ms: 1 << 20,
             "friday_attn_paged_workspace_bytes": lambda b, hq, ms: 1 << 20,
             "friday_gemm_q8_workspace_bytes": lambda t, k, n: 1 << 20,
             "friday_q8_row_bytes": lambda kind, k: k}

    def __init__(self, hip):
        self.hip = hip

    def friday_attn_last_error(self):
        return b""

    def __getattr__(self, name):
        if name in self.SIZES:
            return self.SIZES[name]

        def launch(*args):
            self.hip.record_launch(args)
            return 0
        return launch


@pytest.fixture
def fake_fa(monkeypatch):
    import friday_attn as fa

    hip = FakeHip()
    monkeypatch.setattr(fa, "_lib", FakeLib(hip))
    monkeypatch.setattr(fa.Hip, "_h", hip)
    monkeypatch.setattr(fa.DeviceBuffer, "_live", set())
    monkeypatch.setattr(fa, "_live_graphs", {})
    monkeypatch.setattr(fa, "_deferred_frees", [])
    return fa, hip


def make_ctx(fa, hip):
    import bench

    cx = object.__new__(bench.Ctx)
    cx.fa = fa
    bk = types.SimpleNamespace()
    bk.fabk_fill_normal_f16 = bk.fabk_fill_normal_bf16 = lambda *a: hip.record_launch(a)
    cx.bk = bk
    cx.stream = fa.Stream()
    return bench, cx


def test_bench_sequence_frees_nothing_a_live_graph_uses(fake_fa):
    fa, hip = fake_fa
    bench, cx = make_ctx(fa, hip)
    args = types.SimpleNamespace(ctx=2048, layers=4, steps=2, warmup=1, stat_replays=3, no_cpu=True, no_check=True,
                                 cpu_seconds=0.0)
    bench.headline(cx, args)
    bench.decode_config(cx, "1", 513, 3, 14, 2, 64, 2, 1, False)
    bench.decode_config(cx, "2", 1024, 2, 32, 8, 128, 2, 1, True)
    for p0 in (0, 1024):
        bench.prefill_config(cx, p0, 2, 1)
    bench.prefill_config(cx, 0, 2, 1, q8=True)
    bench.prefill_config(cx, 0, 2, 1, bf16=True)
    bench.paged_config(cx, 2, 1, L=2)
    for T in (1, 512):
        bench.append_config(cx, T, 2, 1)
        bench.append_q8_config(cx, T, 2, 1)
    bench.prefill_vs_decode_config(cx, 1024, 2, 1)
    bench.q8_config(cx, 2048, 2, 2, 1)
    bench.gemv_config(cx, *bench.GEMV_CASES[0], 2, 1)
    bench.layer_block_config(cx, 2048, 2, 2, 1)
    assert hip.violations == []
    # every graph and event the measurements made is gone, and every buffer is freed
    assert hip.execs == {} and hip.graphs == {}
    assert hip.events == set()
    assert hip.allocs == {}


def test_fake_catches_a_free_under_a_live_graph(fake_fa):
    """The checks have teeth: a graph kept alive across a free is refused by the Python
    guard, and seen by the fake when the guard is bypassed."""
    fa, hip = fake_fa
    st = fa.Stream()
    buf = fa.DeviceBuffer(4096)
    g = fa.Graph(st, lambda: fa.decodeWorkspaceInit(buf, stream=st.s))
    with pytest.raises(RuntimeError, match="live Graph"):
        buf.free()
    assert buf.ptr is not None
    hip.hipFree(buf.ptr)  # behind the guard's back
    assert hip.violations and "live graph" in hip.violations[0]
    g.destroy()
    with pytest.raises(RuntimeError, match="after destroy"):
        g.launch()


def test_graph_context_manager_releases(fake_fa):
    fa, hip = fake_fa
    st = fa.Stream()
    buf = fa.DeviceBuffer(4096)
    with fa.Graph(st, lambda: fa.decodeWorkspaceInit(buf, stream=st.s)) as g:
        g.launch()
    assert hip.execs == {} and hip.graphs == {}
    buf.free()
    st.destroy()
    assert hip.violations == [] and hip.allocs == {} and hip.streams == set()


def test_collected_buffer_freed_after_its_graph(fake_fa):
    """A buffer collected while a live graph captured it is not freed then, but as soon as
    that graph is destroyed."""
    import gc

    fa, hip = fake_fa
    st = fa.Stream()
    buf = fa.DeviceBuffer(4096)
    ptr = buf.ptr
    g = fa.Graph(st, lambda: fa.decodeWorkspaceInit(buf, stream=st.s))
    del buf
    gc.collect()
    assert ptr in hip.allocs and hip.violations == []
    g.destroy()
    assert ptr not in hip.allocs and hip.violations == []

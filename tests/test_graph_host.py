"""Host logic of graph capture, without a GPU: the order in which
HipGraphRunner warms up and records the buckets, and the rule that a
workspace a recorded graph holds is never freed.  torch.cuda's graph objects
are replaced by fakes that record what happens; the decode and sampler
workspaces live on the CPU, sized by the library's own size queries (pure
host arithmetic).  A graph "holds" the data pointer of every workspace its
body touched while it was being recorded; the tests check that each such
pointer still belongs to a live tensor after every later capture and growth.
"""
import contextlib

import pytest
import torch

from xvllm import _C
from xvllm import sampler as samp_mod
from xvllm.cuda_graph import HipGraphRunner
from xvllm.layers import attention as attn_mod


class _Recorder:
    def __init__(self):
        self.events = []
        self.capturing = None
        self.held = {}  # bucket -> data pointers its graph holds


@pytest.fixture()
def fake_cuda(monkeypatch):
    rec = _Recorder()

    class FakeGraph:
        def __init__(self):
            self.bs = None

        def pool(self):
            return "pool"

        def replay(self):
            rec.events.append(("replay", self.bs))

    @contextlib.contextmanager
    def fake_graph(graph, pool=None, **kw):
        rec.capturing = graph
        try:
            yield
        finally:
            rec.capturing = None

    monkeypatch.setattr(torch.cuda, "CUDAGraph", FakeGraph)
    monkeypatch.setattr(torch.cuda, "graph", fake_graph)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda *a, **k: None)
    # fresh workspace registries for the test
    monkeypatch.setattr(attn_mod, "_WORKSPACE", {})
    monkeypatch.setattr(attn_mod, "_RETIRED", [])
    monkeypatch.setattr(samp_mod, "_WORKSPACE", {})
    monkeypatch.setattr(samp_mod, "_RETIRED", [])
    return rec


def _live_ptrs():
    ts = list(attn_mod._WORKSPACE.values()) + attn_mod._RETIRED
    ts += list(samp_mod._WORKSPACE.values()) + samp_mod._RETIRED
    return {t.data_ptr() for t in ts}


@pytest.fixture(scope="module")
def lib():
    if not _C.lib_path().exists():
        pytest.fail("libxv_kernels.so is not built (run __graft_entry__.build())")
    return _C.lib()


def _body_factory(rec, lib, dev, vocab=151936, max_blocks=2048):
    def body(bs):
        dws = attn_mod.decode_workspace(dev, lib.xv_paged_decode_workspace_size(bs, 32, 8, max_blocks, 16, 128))
        sws = samp_mod._workspace(dev, lib.xv_sampler_workspace_size(bs, vocab))
        if rec.capturing is not None:
            rec.capturing.bs = bs
            rec.events.append(("capture", bs))
            rec.held[bs] = (dws.data_ptr(), sws.data_ptr())
        else:
            rec.events.append(("eager", bs))
        return bs

    return body


def test_capture_order_largest_first_eager_before_each(fake_cuda, lib):
    """Every bucket runs once eagerly right before its capture, largest first,
    so workspaces reach their final size before the first graph is recorded."""
    dev = torch.device("cpu")
    runner = HipGraphRunner(HipGraphRunner.make_bs_list(256), dev)
    runner.capture(_body_factory(fake_cuda, lib, dev))
    buckets = sorted(runner.bs_list, reverse=True)
    want = [e for bs in buckets for e in (("eager", bs), ("capture", bs))]
    assert fake_cuda.events == want
    # one workspace each: sized by the largest bucket, never regrown
    assert len({p for p in fake_cuda.held.values()}) == 1
    assert attn_mod._RETIRED == [] and samp_mod._RETIRED == []


def test_graphs_keep_their_workspaces_alive_after_growth(fake_cuda, lib):
    """Buckets recorded smallest first (the order that regrows the
    workspaces), then a larger call after capture: every pointer any graph
    recorded still belongs to a live tensor, so no replay lands on freed
    memory."""
    dev = torch.device("cpu")
    body = _body_factory(fake_cuda, lib, dev)
    runner = HipGraphRunner([1, 8, 64], dev)
    runner.bs_list = [64, 8, 1]  # reversed() in capture: 1, 8, 64, smallest first
    runner.capture(body)
    assert [e for e in fake_cuda.events if e[0] == "capture"] == [("capture", 1), ("capture", 8), ("capture", 64)]
    assert len(attn_mod._RETIRED) >= 1 and len(samp_mod._RETIRED) >= 1  # the growth happened
    body(256)  # grows both again, outside any capture
    live = _live_ptrs()
    for bs, ptrs in fake_cuda.held.items():
        for p in ptrs:
            assert p in live, f"graph of bucket {bs} holds a freed workspace"


def test_reserve_sampler_workspace_covers_every_bucket(fake_cuda, lib):
    """reserve_workspace(max_bs) sizes the sampler workspace once: no bucket
    up to max_bs grows it afterwards."""
    dev = torch.device("cpu")
    ws = samp_mod.reserve_workspace(dev, 256, 151936)
    for bs in HipGraphRunner.make_bs_list(256):
        assert samp_mod._workspace(dev, lib.xv_sampler_workspace_size(bs, 151936)) is ws
    assert samp_mod._RETIRED == []


def test_read_samples_rejects_out_of_range_ids():
    """The host check on ids read back: an id outside [0, vocab) raises before
    it can be fed back to the embedding gather."""
    from xvllm.model_runner import ModelRunner, SampledIdOutOfRange

    class Ev:
        def synchronize(self):
            pass

    from collections import deque

    r = ModelRunner.__new__(ModelRunner)
    r.vocab_size = 1000
    r._readback = [(torch.tensor([5, 999, 0, 3], dtype=torch.int64), Ev()), (torch.zeros(4, dtype=torch.int64), Ev())]
    r._pending = deque([(0, 1, 3)])
    assert r.read_samples(1, 3) == ([3], [5, 999, 0])
    with pytest.raises(RuntimeError, match="no launched step"):
        r.read_samples(1, 3)
    r._pending = deque([(0, 1, 3)])
    with pytest.raises(ValueError, match="oldest waiting step"):
        r.read_samples(2, 2)
    for bad in (1000, -1, 1 << 40):
        r._readback[1] = (torch.tensor([5, bad, 0, 3], dtype=torch.int64), Ev())
        r._pending = deque([(1, 2, 2)])
        with pytest.raises(SampledIdOutOfRange):
            r.read_samples(2, 2)


def test_cached_workspaces_are_plain_tensors_after_inference_mode():
    """A per-device workspace first grown inside torch.inference_mode (the
    runner's decode) is a plain tensor: callers outside inference mode can
    still write to it (a test that fills it with NaN patterns does)."""
    import torch

    from xvllm.layers import attention as A
    from xvllm import sampler as Sm

    dev = torch.device("cpu")
    for fn, store in ((A.decode_workspace, A._WORKSPACE), (Sm._workspace, Sm._WORKSPACE)):
        key = (dev.type, dev.index)
        saved = store.pop(key, None)
        try:
            with torch.inference_mode():
                ws = fn(dev, 4096)
            assert not ws.is_inference()
            ws.fill_(255)
        finally:
            store.pop(key, None)
            if saved is not None:
                store[key] = saved

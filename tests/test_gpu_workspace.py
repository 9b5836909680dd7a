"""The per-stream GEMM workspace under graph capture and several host threads
(needs an MI355X).

A workspace buffer, once handed out, stays allocated until the process ends:
a graph captured earlier keeps the pointer it recorded, and another thread
may have looked the buffer up without having enqueued its kernel yet.  So a
larger call on the same stream moves the stream to a new, larger buffer and
leaves the old one alone.
"""
import threading

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    if not _t.cuda.is_available():
        pytest.skip("no GPU")
    return _t


@pytest.fixture(scope="module")
def okq(torch):
    from ocelotl_amd import okq as _okq
    _okq.call("okq_init", 0)
    return _okq


def _problem(torch, orc, seed, t, rows, n, k):
    wq = orc.quantize(t, orc.normal(seed, n * k, 0.02))
    x = orc.normal(seed + 1, rows * k, 1.0)
    return (t, rows, n, k, wq, torch.from_numpy(x).cuda(), torch.from_numpy(wq).cuda())


def _launch(okq, prob, out, stream):
    t, rows, n, k, wq, xd, wd = prob
    okq.call("okq_linear_out_by_in_q", xd.data_ptr(), rows, k, t, wd.data_ptr(), wq.size, n, None, out.data_ptr(),
             stream)


def test_graph_captured_before_the_workspace_grows_replays_correctly(torch, okq, orc):
    """Capture a batch-8 decode call (split-K partials in the workspace), then
    run larger eager calls on the same stream (the workspace grows), then
    replay the graph: every replay equals the eager result bit for bit."""
    s = torch.cuda.Stream()
    small = _problem(torch, orc, 9000, O.Q4_K, 8, 14336, 4096)
    big = [_problem(torch, orc, 9010, O.Q4_K, 32, 14336, 4096), _problem(torch, orc, 9020, O.Q6_K, 300, 4096, 4096)]
    ref = torch.empty(8 * 14336, dtype=torch.float32, device="cuda")
    out = torch.empty_like(ref)
    with torch.cuda.stream(s):
        _launch(okq, small, ref, s.cuda_stream)  # allocates the stream's workspace before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _launch(okq, small, out, s.cuda_stream)
    big_outs = [torch.empty(p[1] * p[2], dtype=torch.float32, device="cuda") for p in big]
    want_big = []
    for p, o in zip(big, big_outs):
        with torch.cuda.stream(s):
            _launch(okq, p, o, s.cuda_stream)  # grows the workspace of this stream
        torch.cuda.synchronize()
        want_big.append(o.cpu().numpy().copy())
    for rep in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert (out.cpu().numpy().view(np.uint32) == ref.cpu().numpy().view(np.uint32)).all(), rep
        for p, o, w in zip(big, big_outs, want_big):  # eager work between the replays
            with torch.cuda.stream(s):
                _launch(okq, p, o, s.cuda_stream)
            torch.cuda.synchronize()
            assert (o.cpu().numpy().view(np.uint32) == w.view(np.uint32)).all(), rep
    del g


def test_two_threads_on_one_stream_growing_its_workspace(torch, okq, orc):
    """Two host threads issue calls of different workspace sizes on one
    stream at the same time (ctypes releases the GIL during each call):
    every result equals the single-threaded one bit for bit."""
    s = torch.cuda.Stream()
    probs = [_problem(torch, orc, 9100, O.Q4_K, 16, 4096, 4096), _problem(torch, orc, 9110, O.Q4_K, 200, 2048, 4096),
             _problem(torch, orc, 9120, O.Q6_K, 24, 8192, 4096), _problem(torch, orc, 9130, O.Q6_K, 520, 1024, 4096)]
    want = []
    for p in probs:
        o = torch.empty(p[1] * p[2], dtype=torch.float32, device="cuda")
        _launch(okq, p, o, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        want.append(o.cpu().numpy().copy())
    reps = 12
    outs = {(i, r): torch.empty(p[1] * p[2], dtype=torch.float32, device="cuda") for i, p in enumerate(probs)
            for r in range(reps)}
    torch.cuda.synchronize()
    errors = []

    def worker(idxs):
        try:
            okq.call("okq_init", 0)
            for r in range(reps):
                for i in idxs:
                    _launch(okq, probs[i], outs[(i, r)], s.cuda_stream)
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=([0, 1],)), threading.Thread(target=worker, args=([3, 2],))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for (i, r), o in outs.items():
        assert (o.cpu().numpy().view(np.uint32) == want[i].view(np.uint32)).all(), (i, r)


def test_graph_replayed_on_another_stream_after_its_capture_stream_is_idle(torch, okq, orc):
    """A graph records its capture stream's workspace pointer.  The rule for
    replays: a replay on another stream must be serialised with the capture
    stream's own work -- here the capture
    stream's eager calls finish (an event the replay stream waits for) before
    the replay starts, and the next eager call on the capture stream waits
    for the replay.  Each replay equals the eager result bit for bit, and so
    do the eager calls in between."""
    cap, other = torch.cuda.Stream(), torch.cuda.Stream()
    prob = _problem(torch, orc, 9200, O.Q4_K, 16, 4096, 14336)  # split-K partials in the workspace
    busy = _problem(torch, orc, 9210, O.Q4_K, 24, 14336, 4096)
    ref = torch.empty(16 * 4096, dtype=torch.float32, device="cuda")
    out = torch.empty_like(ref)
    bo = torch.empty(24 * 14336, dtype=torch.float32, device="cuda")
    with torch.cuda.stream(cap):
        _launch(okq, prob, ref, cap.cuda_stream)
        _launch(okq, busy, bo, cap.cuda_stream)
    torch.cuda.synchronize()
    want_busy = bo.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        _launch(okq, prob, out, cap.cuda_stream)
    for rep in range(3):
        out.fill_(float("nan"))
        with torch.cuda.stream(cap):
            _launch(okq, busy, bo, cap.cuda_stream)  # eager work on the capture stream's workspace
        done = torch.cuda.Event()
        done.record(cap)
        other.wait_event(done)  # serialised: the replay waits for it
        with torch.cuda.stream(other):
            g.replay()
        replayed = torch.cuda.Event()
        replayed.record(other)
        cap.wait_event(replayed)  # and the capture stream waits for the replay
        torch.cuda.synchronize()
        assert (out.cpu().numpy().view(np.uint32) == ref.cpu().numpy().view(np.uint32)).all(), rep
        assert (bo.cpu().numpy().view(np.uint32) == want_busy.view(np.uint32)).all(), rep
    del g

"""ltxk.StreamEvent (GPU): a wait orders the consumer stream's later work after
the producer stream's recorded work, eagerly and inside a captured HIP graph
(replayed several times, with eager work between the replays)."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ltxk():
    import ltxk

    ltxk.load()
    return ltxk


def test_wait_orders_after_a_slow_producer():
    ltxk = _ltxk()
    main, side = torch.cuda.current_stream(), torch.cuda.Stream()
    x = torch.zeros(1 << 20, device="cuda")
    ev = ltxk.StreamEvent()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        torch.cuda._sleep(50_000_000)  # the producer is still asleep when main enqueues its read
        x.fill_(1.0)
        ev.record(side)
    ev.wait(main)
    y = x * 2.0
    x.record_stream(main)
    assert torch.equal(y, torch.full_like(x, 2.0))
    # the same event re-recorded: a later wait takes the latest record
    with torch.cuda.stream(side):
        torch.cuda._sleep(50_000_000)
        x.fill_(3.0)
        ev.record(side)
    ev.wait(main)
    assert torch.equal(x * 1.0, torch.full_like(x, 3.0))


def test_fork_and_join_in_a_captured_graph():
    ltxk = _ltxk()
    side = torch.cuda.Stream()
    fork, join = ltxk.StreamEvent(), ltxk.StreamEvent()
    a = torch.randn(1 << 18, device="cuda")
    b = torch.empty_like(a)
    c = torch.empty_like(a)
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=cap):
        fork.record(cap)
        fork.wait(side)
        with torch.cuda.stream(side):
            torch.cuda._sleep(20_000_000)
            torch.mul(a, 3.0, out=b)
            join.record(side)
        join.wait(cap)
        torch.add(b, 1.0, out=c)
    for i in range(3):
        a.normal_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, a * 3.0 + 1.0), i

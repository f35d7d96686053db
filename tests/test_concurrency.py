"""Concurrent use (GPU): several host threads, each on its own stream, run forward + backward
steps of different size classes at once and get the same bits as one thread alone.

The library keeps no state across calls apart from a thread-local error message, launches on the
caller's stream and allocates nothing, so concurrent calls on different streams must not see each
other.  The reference's operator launches the same way: on the current stream
(csrc/matrix_exp.cu:16) under a device guard (:60), with no global state.
"""

import threading

import pytest
import torch

import flash_hypercons as fh

pytestmark = pytest.mark.gpu


def _step(x, g):
    xi = x.detach().requires_grad_()
    y = fh.matrix_exp(xi)
    (d,) = torch.autograd.grad(y, xi, g)
    return y.detach(), d


def test_threads_on_their_own_streams_match_a_single_thread():
    gen = torch.Generator().manual_seed(5)
    cases = []
    # One case per kernel family: P = 4 (FP32 DMA / BF16 count-ordered), P = 8, P = 16, P = 32.
    for n, dtype, batch in ((4, torch.float32, 8192), (4, torch.bfloat16, 8192), (8, torch.float32, 2048),
                            (16, torch.float32, 512), (32, torch.float16, 128)):
        x = (torch.randn(batch, n, n, generator=gen) / n**0.5).to(dtype).cuda()
        g = torch.randn(batch, n, n, generator=gen).to(dtype).cuda()
        cases.append((x, g))
    want = [_step(x, g) for x, g in cases]
    torch.cuda.synchronize()

    start = threading.Barrier(len(cases))
    failures = []

    def worker(i):
        try:
            stream = torch.cuda.Stream()  # default priority
            x, g = cases[i]
            start.wait()
            with torch.cuda.stream(stream):
                for _ in range(25):
                    y, d = _step(x, g)
            stream.synchronize()
            if not (torch.equal(y, want[i][0]) and torch.equal(d, want[i][1])):
                failures.append(f"case {i}: results differ from the single-thread run")
        except Exception as exc:  # reported below, with the case
            failures.append(f"case {i}: {exc!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not failures, failures

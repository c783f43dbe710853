"""q3_gemm_nt_group_argmax_noalloc (the entry point that never allocates)
against q3_gemm_nt_group_argmax, through the C ABI.

Two calls in a row on the same stream, the second with fewer rows and
columns than the first, so the second runs over key slots the first left
behind: (best, bidx) must equal the allocating entry point's bit for bit,
and both must equal the oracle's argmax of the logits.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from conftest import bits_equal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from q3ops import ops  # noqa: E402

F = np.float32


def note(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_both(rng, M, N, K=1024, group=256):
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    b = rng.integers(-127, 128, (N, K)).astype(np.int8)
    as_ = rng.uniform(1e-3, 1e-1, (M, K // group)).astype(F)
    bs = rng.uniform(1e-3, 1e-1, N).astype(F)
    ta, tas, tb, tbs = dev(a), dev(as_), dev(b), dev(bs)
    outs = []
    for fn in (ops.gemm_nt_group_argmax, ops.gemm_nt_group_argmax_noalloc):
        best = torch.full((M,), -3.0e38, dtype=torch.float32, device="cuda")
        bidx = torch.full((M,), -1, dtype=torch.int32, device="cuda")
        fn(ta, tas, tb, tbs, best, bidx, group)
        torch.cuda.synchronize()
        outs.append((best.cpu().numpy(), bidx.cpu().numpy()))
    logits = oracle.gemm_nt_group(a, as_, b, bs, group)
    return outs, logits


@pytest.mark.parametrize("first,second", [((64, 151936), (1, 151936)),
                                          ((200, 151936), (5, 4096)),
                                          ((16, 151936), (3, 1024))])
def test_noalloc_matches_allocating_entry(cuda, first, second):
    rng = np.random.default_rng(first[0] * 31 + second[0])
    for M, N in (first, second):
        note(f"argmax noalloc vs allocating: M={M} N={N}")
        ((ab, ai), (nb, ni)), logits = run_both(rng, M, N)
        assert np.array_equal(ni, ai), (M, N, ni[:8], ai[:8])
        assert bits_equal(nb, ab), (M, N)
        assert ai.tolist() == [int(i) for i in np.argmax(logits, axis=1)], (M, N)
        assert bits_equal(ab, logits.max(axis=1)), (M, N)


def test_noalloc_under_graph_capture_fresh_stream(cuda):
    """The entry point inside a HIP graph captured on a stream that never ran
    an argmax (an allocation there would break the capture), replayed twice
    with (best, bidx) reset eagerly in between, each replay against the
    oracle; then a smaller eager call on the same device."""
    rng = np.random.default_rng(7)
    M, N, K, group = 4, 151936, 1024, 256
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    b = rng.integers(-127, 128, (N, K)).astype(np.int8)
    as_ = rng.uniform(1e-3, 1e-1, (M, K // group)).astype(F)
    bs = rng.uniform(1e-3, 1e-1, N).astype(F)
    logits = oracle.gemm_nt_group(a, as_, b, bs, group)
    ta, tas, tb, tbs = dev(a), dev(as_), dev(b), dev(bs)
    best = torch.full((M,), -3.0e38, dtype=torch.float32, device="cuda")
    bidx = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    note("argmax noalloc captured on a fresh stream")
    with torch.cuda.graph(graph, stream=st):
        ops.gemm_nt_group_argmax_noalloc(ta, tas, tb, tbs, best, bidx, group, stream=st)
    for rep in range(2):
        best.fill_(-3.0e38)
        bidx.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert bidx.cpu().numpy().tolist() == [int(i) for i in np.argmax(logits, axis=1)], rep
        assert bits_equal(best.cpu().numpy(), logits.max(axis=1)), rep
    (ab, ai), (nb, ni) = run_both(rng, 2, 4096)[0]
    assert np.array_equal(ni, ai) and bits_equal(nb, ab)

"""fmx_fwd_noalloc (the allocation-free fmx_fwd) against fmx_fwd through the C ABI.

Each case needs scratch (fmx_fwd_workspace_bytes > 0): a query of several
passes over per-query docs (streaming kernel), a query of several passes at
d = 1024 (split-d kernel), queries straddling row blocks (tiled kernel), and
d > 4096 (similarity chunks, fewer items per chunk in the scratch).
Two calls in a row, the second smaller, must each give scores bit-identical
to fmx_fwd's on the same inputs: both run the same kernels in the same order,
one with a caller workspace and one with the library's static scratch.
"""

from __future__ import annotations

import pytest
import torch

from conftest import sim
from flash_maxsim_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"

CASES = {
    # name: [(Nq, Lq, B, Ld, d, shared_docs), second smaller call]
    "stream_passes": [(3, 300, 40, 90, 128, 0), (2, 200, 17, 50, 128, 0)],
    "splitd_passes": [(1, 300, 20, 70, 1024, 1), (1, 150, 9, 33, 1024, 1)],
    "tiled_straddle": [(3, 700, 30, 90, 128, 1), (2, 650, 11, 40, 128, 1)],
    # d > 4096: similarity chunks; fmx_fwd's workspace holds all 70 items, the
    # scratch 64 per chunk (256 KB each), so the noalloc call runs two chunks
    "wide_chunks": [(1, 128, 70, 512, 4104, 1), (1, 64, 20, 100, 5000, 1)],
}


def run(lib, Q, D, lengths, scores, Nq, B, Lq, Ld, d, shared, noalloc):
    args = [_lib.FMX_DTYPE_F16, Q.data_ptr(), Q.stride(0), Q.stride(1), D.data_ptr(), D.stride(0), D.stride(1),
            lengths.data_ptr(), scores.data_ptr(), scores.stride(0), scores.stride(1), None,
            Nq, B, Lq, Ld, d, shared]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.fmx_fwd_noalloc(*args, stream)
    else:
        nbytes = lib.fmx_fwd_workspace_bytes(Nq, B, Lq, Ld, d)
        ws = _lib.workspace(nbytes, torch.device(DEV))
        rc = lib.fmx_fwd(*args, _lib.ptr(ws), nbytes, stream)
    _lib.check(rc)


@pytest.mark.parametrize("name", list(CASES))
def test_noalloc_matches_fmx_fwd(name):
    lib = _lib.load()
    for i, (Nq, Lq, B, Ld, d, shared) in enumerate(CASES[name]):
        assert lib.fmx_fwd_workspace_bytes(Nq, B, Lq, Ld, d) > 0, "case must use scratch"
        rows = B if shared else Nq * B
        Q = sim((Nq, Lq, d), 10 * i + Lq).to(DEV)
        D = sim((rows, Ld, d), 10 * i + Ld).to(DEV)
        g = torch.Generator().manual_seed(i + B)
        lengths = torch.randint(0, Ld + 4, (rows,), generator=g, dtype=torch.int32).to(DEV)
        want = torch.full((Nq, B), 7.0, device=DEV)
        got = torch.full((Nq, B), -7.0, device=DEV)
        run(lib, Q, D, lengths, want, Nq, B, Lq, Ld, d, shared, False)
        run(lib, Q, D, lengths, got, Nq, B, Lq, Ld, d, shared, True)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{name} call {i}: max diff {(got - want).abs().max().item()}"


def test_noalloc_graph_replays():
    """fmx_fwd_noalloc captured into a HIP graph on a side stream (after an
    eager call on the device has looked up the scratch address), replayed three
    times with eager work between the replays, among it an eager noalloc call
    on other inputs that rewrites the shared scratch: each replay must give
    fmx_fwd's scores bit for bit."""
    lib = _lib.load()
    Nq, Lq, B, Ld, d, shared = 3, 700, 30, 90, 128, 1  # tiled kernel, queries straddling row blocks
    Q = sim((Nq, Lq, d), 501).to(DEV)
    D = sim((B, Ld, d), 502).to(DEV)
    lengths = torch.randint(0, Ld + 4, (B,), generator=torch.Generator().manual_seed(503), dtype=torch.int32).to(DEV)
    want = torch.empty(Nq, B, device=DEV)
    run(lib, Q, D, lengths, want, Nq, B, Lq, Ld, d, shared, False)
    Q2 = sim((2, 650, d), 504).to(DEV)
    other = torch.empty(2, B, device=DEV)
    run(lib, Q2, D, lengths, other, 2, B, 650, Ld, d, shared, True)  # eager: looks up the scratch
    torch.cuda.synchronize()
    got = torch.full((Nq, B), -7.0, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        run(lib, Q, D, lengths, got, Nq, B, Lq, Ld, d, shared, True)
    torch.cuda.synchronize()
    for r in range(3):
        got.fill_(-7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {r}: max diff {(got - want).abs().max().item()}"
        again = torch.empty(2, B, device=DEV)
        run(lib, Q2, D, lengths, again, 2, B, 650, Ld, d, shared, True)  # eager work in between
        torch.cuda.synchronize()
        assert torch.equal(again, other)

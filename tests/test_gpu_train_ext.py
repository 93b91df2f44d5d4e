"""GPU parity of the training extensions: doc lengths and batched queries.

flash_maxsim_train(Q, D, doc_lengths) and flash_maxsim_train_batched(Q, D,
doc_lengths) against the oracle (scores, the argmax the forward saves, and
the backward formula applied to that argmax: oracle.bwd per query, summed over
queries for dD), and against float64 autograd through the reference's own
naive MaxSim (maxsim_naive) on the CPU, which fixes what an empty doc
contributes (no gradient). Tolerances as in test_gpu_parity.py: scores
within 1e-2 of the oracle, the saved argmax exact up to its tie rule,
gradients within rtol 2e-3 + atol 1e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flash_maxsim_amd as fm
from conftest import sim, to_np32
from flash_maxsim_amd.flash_maxsim import _launch_fwd, _prep
from test_gpu_parity import assert_argmax

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATOL = 1e-2


def saved_argmax(Qn, Dn, lengths, dtype=torch.float16):
    Q3 = Qn if Qn.ndim == 3 else Qn[None]
    Nq, Lq, d = Q3.shape
    B, Ld = Dn.shape[:2]
    Qk = _prep(torch.from_numpy(Q3).to(dtype).to(DEV), dtype)
    Dk = _prep(torch.from_numpy(Dn).to(dtype).to(DEV), dtype)
    lt = None if lengths is None else torch.as_tensor(lengths, dtype=torch.int32, device=DEV)
    _, am = _launch_fwd(Qk, Dk, lt, Nq, B, Lq, Ld, d, True, True)
    return am.cpu().numpy().reshape(Nq, B, Lq)


def reference_grads(oracle_mod, Qn, Dn, am, g, lengths):
    """dQ [Nq, Lq, d], dD [B, Ld, d] in float64 from the oracle's backward,
    with empty docs' upstream gradient set to zero (they give no gradient)."""
    Q3 = Qn if Qn.ndim == 3 else Qn[None]
    g2 = np.array(g, dtype=np.float64).reshape(Q3.shape[0], -1)
    if lengths is not None:
        g2[:, np.asarray(lengths) <= 0] = 0.0
    dQ = np.zeros(Q3.shape)
    dD = np.zeros(Dn.shape)
    for qi in range(Q3.shape[0]):
        a, b = oracle_mod.bwd(Q3[qi], Dn, am[qi], g2[qi])
        dQ[qi] = a
        dD += b
    return dQ, dD


@pytest.mark.parametrize("B, Lq, Ld, d", [(12, 32, 70, 128), (8, 300, 40, 128), (6, 64, 90, 1024), (9, 16, 33, 96)])
def test_train_with_doc_lengths(oracle_mod, B, Lq, Ld, d):
    Q = sim((Lq, d), 1100 + d)
    D = sim((B, Ld, d), 1101 + Lq)
    lengths = torch.randint(1, Ld + 1, (B,), generator=torch.Generator().manual_seed(B), dtype=torch.int32)
    lengths[1] = 0
    lengths[2] = Ld + 7  # clamps to Ld
    Qg, Dg = Q.to(DEV).requires_grad_(True), D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg, lengths.to(DEV))
    g = torch.linspace(-1.0, 2.0, B)
    (s.masked_fill(torch.isinf(s), 0.0) * g.to(DEV)).sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    ref = oracle_mod.maxsim(Qn, Dn, lengths.numpy())[0]
    got = s.detach().double().cpu().numpy()
    np.testing.assert_array_equal(np.isinf(got), np.isinf(ref))
    assert np.abs(got[np.isfinite(ref)] - ref[np.isfinite(ref)]).max() <= ATOL
    am = saved_argmax(Qn, Dn, lengths.numpy())
    clamped = np.clip(lengths.numpy(), 0, Ld)
    for b in range(B):
        if clamped[b] > 0:
            assert (am[0, b] < clamped[b]).all()
    _, am_ref, best = oracle_mod.maxsim(Qn, Dn, lengths.numpy(), want_argmax=True)
    assert_argmax(torch.from_numpy(am), am_ref, best, Qn, Dn, d, lengths.numpy())
    dQ_ref, dD_ref = reference_grads(oracle_mod, Qn, Dn, am, g.numpy(), clamped)
    np.testing.assert_allclose(Qg.grad.double().cpu().numpy(), dQ_ref[0], rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(Dg.grad.double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)
    assert not Dg.grad[1].any()  # the empty doc gets no gradient


@pytest.mark.parametrize("Nq, B, Lq, Ld, d", [
    (3, 10, 32, 60, 128), (16, 20, 32, 40, 128), (4, 6, 100, 50, 1024), (2, 7, 24, 30, 64),
    # Nq*Lq >= 8192: the dD index sorts each doc's entries in chunks of 8192
    (70, 6, 128, 64, 128),      # 8960 entries, two chunks
    (64, 5, 300, 40, 128),      # 19200 entries, three chunks (tiled forward)
    (70, 4, 128, 9, 64),        # 9 rows: every row's entries straddle both chunks
])
def test_train_batched(oracle_mod, Nq, B, Lq, Ld, d):
    Q = sim((Nq, Lq, d), 1200 + Nq)
    D = sim((B, Ld, d), 1201 + d)
    lengths = torch.randint(0, Ld + 1, (B,), generator=torch.Generator().manual_seed(Nq), dtype=torch.int32)
    lengths[0] = 0
    Qg, Dg = Q.to(DEV).requires_grad_(True), D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train_batched(Qg, Dg, lengths.to(DEV))
    assert s.shape == (Nq, B)
    g = torch.randn(Nq, B, generator=torch.Generator().manual_seed(7))
    (s.masked_fill(torch.isinf(s), 0.0) * g.to(DEV)).sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    ref = oracle_mod.maxsim(Qn, Dn, lengths.numpy())
    got = s.detach().double().cpu().numpy()
    np.testing.assert_array_equal(np.isinf(got), np.isinf(ref))
    assert np.abs(got[np.isfinite(ref)] - ref[np.isfinite(ref)]).max() <= ATOL
    # scores equal the batched forward's
    np.testing.assert_array_equal(s.detach().cpu().numpy(),
                                  fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV)).cpu().numpy())
    am = saved_argmax(Qn, Dn, lengths.numpy())
    _, am_ref, best = oracle_mod.maxsim(Qn, Dn, lengths.numpy(), want_argmax=True)
    assert_argmax(torch.from_numpy(am), am_ref, best, Qn, Dn, d, lengths.numpy())
    dQ_ref, dD_ref = reference_grads(oracle_mod, Qn, Dn, am, g.numpy(), lengths.numpy())
    np.testing.assert_allclose(Qg.grad.double().cpu().numpy(), dQ_ref, rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(Dg.grad.double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


def test_train_lengths_match_naive_autograd():
    """Float64 autograd through maxsim_naive on the CPU (the reference's own
    oracle function) fixes the gradients, empty doc included."""
    Q = sim((20, 64), 1300)
    D = sim((7, 30, 64), 1301)
    lengths = torch.tensor([30, 0, 1, 17, 29, 5, 30], dtype=torch.int32)
    Qd, Dd = Q.double().requires_grad_(True), D.double().requires_grad_(True)
    ref = fm.maxsim_naive(Qd, Dd, lengths)
    fin = torch.isfinite(ref)
    (ref[fin] * torch.arange(1.0, 1.0 + int(fin.sum()), dtype=torch.float64)).sum().backward()
    Qg, Dg = Q.to(DEV).requires_grad_(True), D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg, lengths.to(DEV))
    sf = torch.isfinite(s)
    assert torch.equal(sf.cpu(), fin)
    (s[sf] * torch.arange(1.0, 1.0 + int(sf.sum()), device=DEV)).sum().backward()
    np.testing.assert_allclose(Qg.grad.double().cpu().numpy(), Qd.grad.numpy(), rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(Dg.grad.double().cpu().numpy(), Dd.grad.numpy(), rtol=2e-3, atol=ATOL)


def test_train_batched_deterministic_and_grad_only_q():
    Q = sim((8, 32, 128), 1400).to(DEV)
    D = sim((30, 64, 128), 1401).to(DEV)
    outs = []
    for _ in range(2):
        Qg, Dg = Q.clone().requires_grad_(True), D.clone().requires_grad_(True)
        fm.flash_maxsim_train_batched(Qg, Dg).sum().backward()
        outs.append((Qg.grad.clone(), Dg.grad.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    Qg = Q.clone().requires_grad_(True)
    fm.flash_maxsim_train_batched(Qg, D).sum().backward()
    assert torch.equal(Qg.grad, outs[0][0])


@pytest.mark.parametrize("B, Lq, Ld, d", [(5, 24, 37, 20), (3, 16, 300, 2048), (40, 8, 9, 8), (3, 40, 50, 4096)])
def test_train_grad_only_d(oracle_mod, B, Lq, Ld, d):
    """dD alone (Q without grad) over shapes that exercise the dD writer's
    row mapping: d % 8 != 0 (scalar stores, 16 rows per wave pass), d = 2048
    (four passes over a row's chunks) and many tiny docs (slabs spanning docs)."""
    Q = sim((Lq, d), 1500 + d)
    D = sim((B, Ld, d), 1501 + d)
    Dg = D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Q.to(DEV), Dg)
    g = torch.linspace(0.5, -1.5, B)
    (s * g.to(DEV)).sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    am = saved_argmax(Qn, Dn, None)
    _, dD_ref = reference_grads(oracle_mod, Qn, Dn, am, g.numpy(), None)
    np.testing.assert_allclose(Dg.grad.double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


@pytest.mark.parametrize("Nq, B, Lq, Ld, d", [(2, 300, 32, 256, 128), (1, 40, 64, 300, 1024)])
def test_bwd_forked_chains_match_separate_chains(Nq, B, Lq, Ld, d):
    """With both gradients asked for and dD of 2^24 bytes or more, fmx_bwd_batched
    runs the dQ chain on a second stream beside the dD chain and joins it to the
    caller's stream. Its outputs must equal, byte for byte, the chains run one at
    a time on the caller's stream (dQ alone, then dD alone: no second stream),
    over calls back to back with changing gradients, each result copied on the
    caller's stream right after its call (a missing join would let the copy read
    an unfinished dQ)."""
    from flash_maxsim_amd import _lib

    assert B * Ld * d * 2 >= 1 << 24
    gen = torch.Generator().manual_seed(1700 + d)
    Qk = _prep(torch.randn(Nq, Lq, d, generator=gen).to(torch.float16).to(DEV), torch.float16)
    Dk = _prep(torch.randn(B, Ld, d, generator=gen).to(torch.float16).to(DEV), torch.float16)
    lengths = torch.randint(1, Ld + 1, (B,), generator=gen, dtype=torch.int32)
    lengths[3] = 0
    lengths[5] = Ld
    lengths = lengths.to(DEV)
    _, am = _launch_fwd(Qk, Dk, lengths, Nq, B, Lq, Ld, d, True, True)
    lib = _lib.load()
    nbytes = lib.fmx_bwd_batched_workspace_bytes(Nq, B, Lq, Ld, d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)

    def call(g, dQ, dD):
        rc = lib.fmx_bwd_batched(
            _lib.dtype_code(Qk), Qk.data_ptr(), Qk.stride(0), Qk.stride(1), Dk.data_ptr(), Dk.stride(0),
            Dk.stride(1), lengths.data_ptr(), am.data_ptr(), g.data_ptr(), g.stride(0), g.stride(1),
            _lib.ptr(dQ), _lib.ptr(dD), Nq, B, Lq, Ld, d, ws.data_ptr(), nbytes,
            torch.cuda.current_stream().cuda_stream,
        )
        _lib.check(rc)

    forked = []
    for it in range(4):
        g = torch.randn(Nq, B, generator=gen).to(DEV)
        dQ = torch.empty(Nq, Lq, d, dtype=torch.float16, device=DEV)
        dD = torch.empty(B, Ld, d, dtype=torch.float16, device=DEV)
        call(g, dQ, dD)
        forked.append((g, dQ.clone(), dD.clone()))
    for g, fQ, fD in forked:
        sQ = torch.empty(Nq, Lq, d, dtype=torch.float16, device=DEV)
        sD = torch.empty(B, Ld, d, dtype=torch.float16, device=DEV)
        call(g, sQ, None)
        call(g, None, sD)
        assert torch.count_nonzero(sQ) > 0 and torch.count_nonzero(sD) > 0
        assert torch.equal(fQ, sQ) and torch.equal(fD, sD)


@pytest.mark.parametrize(
    "Nq, B, Lq, Ld, d",
    [(1, 9, 100, 7, 300), (3, 5, 100, 6, 1100), (4, 4, 128, 5, 520), (1, 3, 513, 9, 264), (2, 6, 40, 3, 128)],
)
def test_bwd_exact_on_integer_grid(Nq, B, Lq, Ld, d):
    """fmx_bwd_batched on a given argmax with many entries per doc row (Ld of 3-9
    rows, up to 513 (query, token) entries per doc), integer Q, D and gradients:
    every fp32 sum is exact, so dD and dQ must equal integer arithmetic, whatever
    the order of the sums. d % 8 != 0 (partial chunks), d > 1024 (rows wider than
    a wave's 64 lanes of 8 elements), several queries, empty docs and ragged
    lengths."""
    from flash_maxsim_amd import _lib

    gen = torch.Generator().manual_seed(1800 + d + Lq)
    Q = torch.randint(-1, 2, (Nq, Lq, d), generator=gen)
    D = torch.randint(-2, 3, (B, Ld, d), generator=gen)
    g = torch.tensor([-1, 1, 2])[torch.randint(0, 3, (Nq, B), generator=gen)]
    lengths = torch.randint(1, Ld + 1, (B,), generator=gen, dtype=torch.int32)
    lengths[1] = 0
    am = torch.minimum(
        torch.randint(0, Ld, (Nq, B, Lq), generator=gen, dtype=torch.int32),
        (lengths.clamp(min=1) - 1)[None, :, None],
    )
    dD_ref = torch.zeros(B, Ld, d, dtype=torch.int64)
    dQ_ref = torch.zeros(Nq, Lq, d, dtype=torch.int64)
    for qi in range(Nq):
        for b in range(B):
            if lengths[b] <= 0:
                continue
            dD_ref[b].index_add_(0, am[qi, b].long(), g[qi, b] * Q[qi])
            dQ_ref[qi] += g[qi, b] * D[b, am[qi, b].long()]
    assert dD_ref.abs().max() <= 2048 and dQ_ref.abs().max() <= 2048

    dp = (d + 7) // 8 * 8  # the C-ABI takes rows padded to a multiple of 8 elements
    Qd = torch.zeros(Nq, Lq, dp, dtype=torch.float16)
    Qd[..., :d] = Q.to(torch.float16)
    Dd = torch.zeros(B, Ld, dp, dtype=torch.float16)
    Dd[..., :d] = D.to(torch.float16)
    Qd, Dd = Qd.to(DEV), Dd.to(DEV)
    gd = g.to(torch.float32).to(DEV)
    amd = am.reshape(Nq * B, Lq).contiguous().to(DEV)
    ld = lengths.to(DEV)
    dQ = torch.full((Nq, Lq, d), float("nan"), dtype=torch.float16, device=DEV)
    dD = torch.full((B, Ld, d), float("nan"), dtype=torch.float16, device=DEV)
    lib = _lib.load()
    nbytes = lib.fmx_bwd_batched_workspace_bytes(Nq, B, Lq, Ld, d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    rc = lib.fmx_bwd_batched(
        _lib.FMX_DTYPE_F16, Qd.data_ptr(), Qd.stride(0), Qd.stride(1), Dd.data_ptr(), Dd.stride(0), Dd.stride(1),
        ld.data_ptr(), amd.data_ptr(), gd.data_ptr(), gd.stride(0), gd.stride(1), dQ.data_ptr(), dD.data_ptr(),
        Nq, B, Lq, Ld, d, ws.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream,
    )
    _lib.check(rc)
    assert torch.equal(dD.cpu().to(torch.int64), dD_ref)
    assert torch.equal(dQ.cpu().to(torch.int64), dQ_ref)


def test_bwd_graph_capture_replays():
    """fmx_bwd_batched captured into a HIP graph at a size that forks the dQ
    chain when run eagerly: under capture both chains stay on the capturing
    stream. Every replay, with eager work and synchronisations between them,
    must equal the eager result byte for byte."""
    from flash_maxsim_amd import _lib

    Nq, B, Lq, Ld, d = 1, 300, 32, 256, 128
    assert B * Ld * d * 2 >= 1 << 24
    gen = torch.Generator().manual_seed(2000)
    Qk = _prep(torch.randn(Nq, Lq, d, generator=gen).to(torch.float16).to(DEV), torch.float16)
    Dk = _prep(torch.randn(B, Ld, d, generator=gen).to(torch.float16).to(DEV), torch.float16)
    lengths = torch.randint(1, Ld + 1, (B,), generator=gen, dtype=torch.int32).to(DEV)
    _, am = _launch_fwd(Qk, Dk, lengths, Nq, B, Lq, Ld, d, True, True)
    g = torch.randn(Nq, B, generator=gen).to(DEV)
    lib = _lib.load()
    nbytes = lib.fmx_bwd_batched_workspace_bytes(Nq, B, Lq, Ld, d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    dQ = torch.empty(Nq, Lq, d, dtype=torch.float16, device=DEV)
    dD = torch.empty(B, Ld, d, dtype=torch.float16, device=DEV)

    def call():
        rc = lib.fmx_bwd_batched(
            _lib.dtype_code(Qk), Qk.data_ptr(), Qk.stride(0), Qk.stride(1), Dk.data_ptr(), Dk.stride(0),
            Dk.stride(1), lengths.data_ptr(), am.data_ptr(), g.data_ptr(), g.stride(0), g.stride(1),
            dQ.data_ptr(), dD.data_ptr(), Nq, B, Lq, Ld, d, ws.data_ptr(), nbytes,
            torch.cuda.current_stream().cuda_stream,
        )
        _lib.check(rc)

    call()
    torch.cuda.synchronize()
    wantQ, wantD = dQ.clone(), dD.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call()
    torch.cuda.synchronize()
    for _ in range(3):
        dQ.fill_(float("nan"))
        dD.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dQ, wantQ) and torch.equal(dD, wantD)
        call()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(dQ, wantQ) and torch.equal(dD, wantD)


def test_bwd_forked_from_two_host_threads():
    """Two host threads, each on its own stream with its own outputs and
    workspace, run the forked backward (dD of 2^24 bytes or more) at the same
    time, several times over: the library's shared second stream and its
    fork/join events must keep every call's dQ ordered before its own stream's
    later work. Each result must equal the serial one byte for byte."""
    import threading

    from flash_maxsim_amd import _lib

    Nq, B, Lq, Ld, d = 1, 300, 32, 256, 128
    gen = torch.Generator().manual_seed(2100)
    Qk = _prep(torch.randn(Nq, Lq, d, generator=gen).to(torch.float16).to(DEV), torch.float16)
    Dk = _prep(torch.randn(B, Ld, d, generator=gen).to(torch.float16).to(DEV), torch.float16)
    lengths = torch.randint(1, Ld + 1, (B,), generator=gen, dtype=torch.int32).to(DEV)
    _, am = _launch_fwd(Qk, Dk, lengths, Nq, B, Lq, Ld, d, True, True)
    grads = [torch.randn(Nq, B, generator=gen).to(DEV) for _ in range(2)]
    lib = _lib.load()
    nbytes = lib.fmx_bwd_batched_workspace_bytes(Nq, B, Lq, Ld, d)

    def call(g, dQ, dD, ws, stream):
        rc = lib.fmx_bwd_batched(
            _lib.dtype_code(Qk), Qk.data_ptr(), Qk.stride(0), Qk.stride(1), Dk.data_ptr(), Dk.stride(0),
            Dk.stride(1), lengths.data_ptr(), am.data_ptr(), g.data_ptr(), g.stride(0), g.stride(1),
            dQ.data_ptr(), dD.data_ptr(), Nq, B, Lq, Ld, d, ws.data_ptr(), nbytes, stream.cuda_stream,
        )
        _lib.check(rc)

    bufs = [(torch.empty(Nq, Lq, d, dtype=torch.float16, device=DEV),
             torch.empty(B, Ld, d, dtype=torch.float16, device=DEV),
             torch.empty(nbytes, dtype=torch.uint8, device=DEV)) for _ in range(2)]
    main = torch.cuda.current_stream()
    want = []
    for i in range(2):
        call(grads[i], *bufs[i], main)
        torch.cuda.synchronize()
        want.append((bufs[i][0].clone(), bufs[i][1].clone()))
    streams = [torch.cuda.Stream() for _ in range(2)]
    got = [[], []]
    errors = []

    def worker(i):
        try:
            torch.cuda.set_device(0)
            with torch.cuda.stream(streams[i]):
                for _ in range(6):
                    bufs[i][0].fill_(float("nan"))
                    bufs[i][1].fill_(float("nan"))
                    call(grads[i], *bufs[i], streams[i])
                    got[i].append((bufs[i][0].clone(), bufs[i][1].clone()))  # ordered after the join
        except Exception as e:  # reported on the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in range(2):
        assert len(got[i]) == 6
        for gQ, gD in got[i]:
            assert torch.equal(gQ, want[i][0]) and torch.equal(gD, want[i][1])

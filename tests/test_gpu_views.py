"""GPU parity of operands read in place: views of padded stores.

The Python API hands a view straight to the kernels when its row strides are
multiples of 8 elements (and at least d), its rows start 16-byte aligned and
it already has the kernel dtype; d % 8 != 0 is then masked in the kernels
instead of padded in a copy. Here the padding of every store holds NaN (uint8
codes: 0xFF), so a kernel that read past d would turn the score NaN or wrong.
Each case goes through a different kernel: the streaming kernel (one query,
two docs per workgroup, per-query docs), the tiled kernel (batched queries; d
= 128 with a 136-element row stride takes its LDS DMA tile path), the split-d
kernel, the training forward and backward, and the uint8 kernel. Scores are
checked against the CPU oracle on the same values (1e-2 absolute), gradients
within 1e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flash_maxsim_amd as fm
from flash_maxsim_amd.flash_maxsim import _prep
from conftest import sim, to_np32
from test_gpu_parity import ATOL, assert_scores

pytestmark = pytest.mark.gpu

DEV = "cuda"


def store_view(x: torch.Tensor, width: int, rows: int | None = None, fill=float("nan")) -> torch.Tensor:
    """x placed in a device store whose rows are `width` wide (and whose docs,
    with rows given, hold `rows` tokens), padding filled with `fill`; returns
    the view of x inside it."""
    shape = list(x.shape)
    shape[-1] = width
    if rows is not None:
        shape[-2] = rows
    store = torch.full(shape, fill, dtype=x.dtype, device=DEV)
    idx = tuple(slice(0, n) for n in x.shape)
    store[idx] = x.to(DEV)
    view = store[idx]
    assert _prep(view, x.dtype) is view, "view should be read in place"
    return view


@pytest.mark.parametrize("Lq, B, Ld, d, width, dtype", [
    (32, 41, 77, 100, 104, torch.float16),    # stream kernel, short docs in pairs, partial 8-chunk
    (32, 9, 300, 124, 128, torch.bfloat16),
    (128, 30, 90, 100, 112, torch.float16),   # long query over short docs: tiled kernel
    (16, 12, 64, 128, 136, torch.float16),    # unmasked width, wider rows
    (32, 12, 64, 300, 312, torch.float16),    # split-d kernel
])
def test_single_query_store_views(oracle_mod, Lq, B, Ld, d, width, dtype):
    Q = sim((Lq, d), 900 + d, dtype)
    D = sim((B, Ld, d), 901 + d, dtype)
    lengths = torch.randint(0, Ld + 2, (B,), generator=torch.Generator().manual_seed(B), dtype=torch.int32)
    lengths[0] = Ld
    Qv = store_view(Q, width)
    Dv = store_view(D, width, rows=Ld + 5)     # doc stride (Ld + 5) * width
    out = fm.flash_maxsim(Qv, Dv, lengths.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0]
    assert_scores(out, ref)


@pytest.mark.parametrize("Nq, Lq, B, Ld, d, width, dtype", [
    (4, 64, 40, 90, 100, 112, torch.float16),   # tiled kernel, masked width
    (3, 128, 30, 100, 128, 136, torch.float16),  # tiled kernel, LDS DMA tiles, 272-byte rows
    (3, 96, 20, 70, 96, 104, torch.bfloat16),
])
def test_batched_store_views(oracle_mod, Nq, Lq, B, Ld, d, width, dtype):
    Q = sim((Nq, Lq, d), 910 + Lq, dtype)
    D = sim((B, Ld, d), 911 + B, dtype)
    out = fm.flash_maxsim_batched(store_view(Q, width, rows=Lq + 3), store_view(D, width))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D))
    assert out.shape == (Nq, B)
    assert_scores(out, ref)


def test_per_query_docs_store_views(oracle_mod):
    Nq, Lq, B, Ld, d = 5, 32, 9, 77, 100
    Q = sim((Nq, Lq, d), 920)
    D = sim((Nq, B, Ld, d), 921)
    lengths = torch.randint(0, Ld + 3, (Nq * B,), generator=torch.Generator().manual_seed(922), dtype=torch.int32)
    out = fm.flash_maxsim_batched(store_view(Q, 104), store_view(D, 104), lengths.to(DEV), shared_docs=False)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D.reshape(Nq * B, Ld, d)), lengths.numpy(), shared_docs=False)
    assert_scores(out, ref)


@pytest.mark.parametrize("Lq, B, Ld, d, width", [(32, 7, 60, 100, 112), (16, 5, 40, 300, 304)])
def test_train_store_views(oracle_mod, Lq, B, Ld, d, width):
    Q = sim((Lq, d), 930 + d)
    D = sim((B, Ld, d), 931 + d)
    g = torch.linspace(-1.0, 2.0, B, dtype=torch.float32)
    Qs = torch.full((Lq, width), float("nan"), dtype=torch.float16, device=DEV)
    Ds = torch.full((B, Ld, width), float("nan"), dtype=torch.float16, device=DEV)
    Qs[:, :d] = Q.to(DEV)
    Ds[:, :, :d] = D.to(DEV)
    Qs.requires_grad_(True)
    Ds.requires_grad_(True)
    s = fm.flash_maxsim_train(Qs[:, :d], Ds[:, :, :d])
    (s * g.to(DEV)).sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    ref, am_ref, _best = oracle_mod.maxsim(Qn, Dn, want_argmax=True)
    assert_scores(s, ref[0])
    # gradients reach the stores' first d columns only
    assert not Qs.grad[:, d:].any() and not Ds.grad[:, :, d:].any()
    dQ_ref, dD_ref = oracle_mod.bwd(Qn, Dn, am_ref, g.numpy())
    np.testing.assert_allclose(Qs.grad[:, :d].double().cpu().numpy(), dQ_ref, rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(Ds.grad[:, :, :d].double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


@pytest.mark.parametrize("d, width", [(100, 112), (100, 104), (120, 128)])
def test_int8_codes_store_views(oracle_mod, d, width):
    B, Lq, Ld = 11, 32, 128
    Q = sim((Lq, d), 940 + d)
    D = sim((B, Ld, d), 941 + d, torch.float32)
    codes, s, m = fm.quantize_int8(D)
    lengths = [128, 0, 16, 15, 77, 1, 128, 100, 64, 65, 2]
    cv = store_view(codes, width, fill=255)
    out = fm.flash_maxsim_int8(store_view(Q.half(), width), cv, s.to(DEV), m.to(DEV),
                               torch.tensor(lengths, dtype=torch.int32, device=DEV))
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(s), to_np32(m), lengths)
    assert_scores(out, ref)

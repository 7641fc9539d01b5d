"""Allocation-free split RVQ encode (fm_rvq_encode_split_noalloc) against the
workspace entry point fm_rvq_encode_split, through the C ABI: codes identical
on two calls in a row, the second with a smaller input (the fixed scratch keeps
the first call's contents), and a clear error past the scratch limit."""

from __future__ import annotations

import pytest
import torch

from fast_mimi_amd import _native as nat

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _codebooks(n, e, d, seed):
    g = torch.Generator().manual_seed(seed)
    embed_sum = (torch.randn(n, e, d, generator=g) / 16).to(DEV)
    usage = torch.ones(n, e, device=DEV)
    emb = torch.empty(n, e, d, device=DEV)
    emb_t = torch.empty(n, d, e, device=DEV)
    norms = torch.empty(n, e, device=DEV)
    for j in range(n):
        nat.call("fm_rvq_prepare_codebook", embed_sum[j].data_ptr(), usage[j].data_ptr(), e, d,
                 1e-5, emb[j].data_ptr(), emb_t[j].data_ptr(), norms[j].data_ptr(), _stream())
    return emb, emb_t, norms


def _encode(noalloc, x, B, T, d, e, nsem, nac, books):
    emb, emb_t, norms = books
    M = B * T
    n = nsem + nac
    codes = torch.full((B, n, T), -1, dtype=torch.int64, device=DEV)
    if noalloc:
        nat.call("fm_rvq_encode_split_noalloc", x.data_ptr(), 2 * d, M, T, d, e, nsem, nac,
                 emb.data_ptr(), emb_t.data_ptr(), norms.data_ptr(), codes.data_ptr(), n * T,
                 _stream())
    else:
        wsb = nat.library().fm_rvq_split_workspace_bytes(M, d, e)
        ws = torch.empty((wsb + 3) // 4, device=DEV)
        nat.call("fm_rvq_encode_split", x.data_ptr(), 2 * d, M, T, d, e, nsem, nac,
                 emb.data_ptr(), emb_t.data_ptr(), norms.data_ptr(), codes.data_ptr(), n * T,
                 ws.data_ptr(), wsb, _stream())
    torch.cuda.synchronize()
    return codes.cpu()


@pytest.mark.parametrize("shapes", [
    ((16, 125, 1, 7, 2048, 256), (1, 125, 1, 7, 2048, 256)),   # C3-sized, then the C2 shape
    ((64, 125, 1, 31, 2048, 256), (3, 40, 1, 5, 2048, 256)),   # C5-sized (8,000 rows), then small
    ((4, 50, 2, 3, 1000, 128), (2, 33, 2, 3, 1000, 128)),      # ragged chunks, other dim
    ((2, 40, 1, 2, 48, 8), (1, 17, 1, 2, 48, 8)),              # general kernel
])
def test_noalloc_split_encode_matches_workspace_entry_point(shapes):
    for i, (B, T, nsem, nac, e, d) in enumerate(shapes):
        books = _codebooks(nsem + nac, e, d, seed=B * T + i)
        g = torch.Generator().manual_seed(7 + i)
        x = (torch.randn(B * T, 2 * d, generator=g) * 0.3).to(DEV)
        want = _encode(False, x, B, T, d, e, nsem, nac, books)
        got = _encode(True, x, B, T, d, e, nsem, nac, books)
        assert ((want >= 0) & (want < e)).all()
        assert torch.equal(got, want), f"call {i}: B={B} T={T}"


def test_noalloc_rejects_inputs_past_the_scratch_limit():
    lib = nat.library()
    limit = lib.fm_rvq_noalloc_scratch_bytes()
    d, e = 256, 2048
    rows = 8_000
    assert lib.fm_rvq_split_workspace_bytes(rows, d, e) <= limit
    big = 9_000
    assert lib.fm_rvq_split_workspace_bytes(big, d, e) > limit
    books = _codebooks(2, e, d, seed=1)
    x = torch.zeros(big, 2 * d, device=DEV)
    codes = torch.empty(1, 2, big, dtype=torch.int64, device=DEV)
    status = lib.fm_rvq_encode_split_noalloc(x.data_ptr(), 2 * d, big, big, d, e, 1, 1,
                                             books[0].data_ptr(), books[1].data_ptr(),
                                             books[2].data_ptr(), codes.data_ptr(), 2 * big, _stream())
    assert status == 1003
    with pytest.raises(nat.NativeError, match="fixed scratch"):
        nat.check(status, "fm_rvq_encode_split_noalloc")

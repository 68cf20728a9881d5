"""matris_csr_build_noalloc (the entry point that allocates nothing) against
matris_csr_build_deferred (the same build with a caller-allocated workspace), both called
through the C-ABI: rowptr and perm must be identical, bit for bit, on two calls in a row
(the second smaller, so stale scratch contents from the first would show), for keys in
arbitrary order (histogram / scan / scatter / per-segment sort through the scratch) and
for ascending keys (perm NULL).  A size beyond the static scratch is refused before any
launch."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
E_SCRATCH = -1006
SCRATCH_BYTES = 48 << 20


def _p(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _keys(R, S, seed, sort=False):
    g = torch.Generator().manual_seed(seed)
    k = torch.randint(0, S, (R,), generator=g, dtype=torch.int32)
    k = torch.where(k % 5 == 2, (k + 1) % S, k)  # some empty segments
    if sort:
        k = torch.sort(k)[0]
    return k.to(DEV)


def _build(lib, keys, S, with_perm, noalloc):
    R = keys.shape[0]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rowptr = torch.full((S + 1,), -7, dtype=torch.int32, device=DEV)
    perm = torch.full((max(R, 1),), -7, dtype=torch.int32, device=DEV) if with_perm else None
    if noalloc:
        rc = lib.matris_csr_build_noalloc(R, _p(keys), 1, S, _p(rowptr), _p(perm), stream)
    else:
        nbytes = lib.matris_csr_workspace_bytes(R, S)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        rc = lib.matris_csr_build_deferred(R, _p(keys), 1, S, _p(rowptr), _p(perm), _p(ws), nbytes, stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return rowptr, (perm[:R] if with_perm else None)


@pytest.mark.parametrize("sort", [False, True])
def test_noalloc_csr_matches_workspace_build_on_two_calls(sort):
    from matris_amd import _lib
    from matris_amd.model import ops
    lib = _lib.load()
    ops.status_take()
    for R, S, seed in ((300_000, 40_000, 1), (5_000, 700, 2)):  # the second call is smaller
        keys = _keys(R, S, seed, sort)
        print(f"noalloc csr: R={R} S={S} sorted={sort}", flush=True)
        a_ptr, a_perm = _build(lib, keys, S, not sort, noalloc=False)
        b_ptr, b_perm = _build(lib, keys, S, not sort, noalloc=True)
        assert torch.equal(a_ptr, b_ptr)
        if not sort:
            assert torch.equal(a_perm, b_perm)
            assert torch.equal(b_perm.cpu().long(), torch.argsort(keys.cpu().long(), stable=True))
        ref_ptr = torch.zeros(S + 1, dtype=torch.int64)
        ref_ptr[1:] = torch.cumsum(torch.bincount(keys.cpu().long(), minlength=S), 0)
        assert torch.equal(b_ptr.cpu().long(), ref_ptr)
    assert ops.status_take() == 0


def test_noalloc_csr_refuses_sizes_beyond_the_scratch():
    from matris_amd import _lib
    from matris_amd.model import ops
    lib = _lib.load()
    keys = _keys(16, 4, 3)
    rowptr = torch.empty(5, dtype=torch.int32, device=DEV)
    perm = torch.empty(16, dtype=torch.int32, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    too_many = SCRATCH_BYTES // 4  # rows alone would need 4 bytes each in the scratch
    assert lib.matris_csr_workspace_bytes(too_many, 4) > SCRATCH_BYTES
    assert lib.matris_csr_build_noalloc(too_many, _p(keys), 1, 4, _p(rowptr), _p(perm), stream) == E_SCRATCH
    assert lib.matris_csr_build_noalloc(-1, _p(keys), 1, 4, _p(rowptr), _p(perm), stream) != 0
    # still usable afterwards
    a_ptr, a_perm = _build(lib, keys, 4, True, noalloc=False)
    b_ptr, b_perm = _build(lib, keys, 4, True, noalloc=True)
    assert torch.equal(a_ptr, b_ptr) and torch.equal(a_perm, b_perm)
    assert ops.status_take() == 0


def test_noalloc_csr_flags_out_of_range_keys_like_the_deferred_build():
    """An out-of-range key is left out and sets STATUS_CSR_KEY, as in the deferred build
    (the key stays inside the int32 range the kernels index with)."""
    from matris_amd import _lib
    from matris_amd.model import ops
    lib = _lib.load()
    ops.status_take()
    keys = _keys(5_000, 300, 4)
    keys[17] = 300
    a_ptr, a_perm = _build(lib, keys, 300, True, noalloc=False)
    assert ops.status_take() == ops.STATUS_CSR_KEY
    b_ptr, b_perm = _build(lib, keys, 300, True, noalloc=True)
    assert ops.status_take() == ops.STATUS_CSR_KEY
    assert torch.equal(a_ptr, b_ptr) and int(b_ptr[-1]) == 4_999
    assert torch.equal(a_perm[:4_999], b_perm[:4_999])

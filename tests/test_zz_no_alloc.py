"""The allocation-free attention entry point (kvp_attn_forward_range_noalloc)
against the allocating one (kvp_attn_forward_range), through the C-ABI.

Both run the same kernels on the same launch plan; only where the split
partials live differs (the library's fixed device scratch array instead of
an allocated workspace), so the outputs must be equal bit for bit. Each case
makes two calls in a row, the second with a smaller input, so the second
call runs over scratch contents the first one left.
"""

import numpy as np
import pytest
import torch

from kvpersist import _lib, api

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qkv(nq, keys, heads, seed, dtype):
    g = torch.Generator(device=DEV).manual_seed(seed)
    D = heads * 128
    q = torch.randn(nq, D, generator=g, device=DEV).to(dtype)
    k = torch.randn(keys, D, generator=g, device=DEV).to(dtype)
    v = torch.randn(keys, D, generator=g, device=DEV).to(dtype)
    return q, k, v


def _both(dtype, nq, keys, heads, key_begin, seed, with_map=False):
    lib = _lib.load()
    D = heads * 128
    dt = api.FP32 if dtype == torch.float32 else api.BF16
    q, k, v = _qkv(nq, keys, heads, seed, dtype)
    arena = kvmap = None
    if with_map:
        rng = np.random.default_rng(seed)
        rows = rng.choice(keys, size=64, replace=False)
        arena = torch.zeros(64, 2 * D, dtype=dtype, device=DEV)
        m = torch.full((keys,), -1, dtype=torch.int64)
        for s, r in enumerate(rows):
            arena[s, :D] = k[int(r)]
            arena[s, D:] = v[int(r)]
            m[int(r)] = s
        kvmap = m.to(DEV)
    ref = torch.empty_like(q)
    got = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    args = (dt, q.data_ptr(), k.data_ptr(), v.data_ptr(),
            arena.data_ptr() if arena is not None else None,
            kvmap.data_ptr() if kvmap is not None else None)
    assert lib.kvp_attn_forward_range(*args, ref.data_ptr(), nq, D, heads, key_begin, keys,
                                      stream) == 0, lib.kvp_last_error()
    assert lib.kvp_attn_forward_range_noalloc(*args, got.data_ptr(), nq, D, heads, key_begin,
                                              keys, stream) == 0, lib.kvp_last_error()
    torch.cuda.synchronize()
    return got, ref, api.attn_splits(dt, nq, heads, 1, keys - key_begin)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_equals_allocating_entry_two_calls(dtype):
    # C3 frame 7: 1560 queries x 12 heads over 12,480 keys (a split launch)
    got, ref, splits = _both(dtype, 1560, 12480, 12, 0, seed=1, with_map=True)
    assert splits > 1
    assert torch.equal(got, ref)
    # second call, smaller: 700 queries x 4 heads over keys [1000, 5000)
    got, ref, splits = _both(dtype, 700, 5000, 4, 1000, seed=2)
    assert splits > 1
    assert torch.equal(got, ref)


def test_noalloc_rejects_bad_arguments_like_the_allocating_entry():
    lib = _lib.load()
    # head_dim != 128 is refused before anything reaches the device
    rc = lib.kvp_attn_forward_range_noalloc(1, 16, 16, 16, None, None, 16, 10, 100, 1, 0, 10,
                                            None)
    assert rc != 0 and b"head_dim" in lib.kvp_last_error()

"""The allocation-free attention entry point (kvp_attn_forward_range_noalloc)
against the allocating one (kvp_attn_forward_range), through the C-ABI.

Both run the same kernels on the same launch plan; only where the split
partials live differs (the library's fixed device scratch array instead of
an allocated workspace), so the outputs must be equal bit for bit. Each case
makes two calls in a row, the second with a smaller input, so the second
call runs over scratch contents the first one left. The allocation-free call
goes first, on a stream no launch has used, and the library's count of
split workspaces must not change across it (had it fallen back to the
allocating path, that stream would now hold one); the allocating call after
it creates that stream's workspace, which kvp_attn_workspace_release frees.
The entry's refusal of partials above its 64 MiB array cannot be reached on
this GPU: a one-frame launch splits only while its workgroups underfill the
CUs x 2 slots, which bounds the fp32 partials at 512 x 128 x 128 x 4 B
(33.5 MB).
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
    torch.cuda.synchronize()
    side = torch.cuda.Stream()  # never used by a launch of this library
    stream = side.cuda_stream
    args = (dt, q.data_ptr(), k.data_ptr(), v.data_ptr(),
            arena.data_ptr() if arena is not None else None,
            kvmap.data_ptr() if kvmap is not None else None)
    n0 = lib.kvp_attn_workspace_count()
    assert lib.kvp_attn_forward_range_noalloc(*args, got.data_ptr(), nq, D, heads, key_begin,
                                              keys, stream) == 0, lib.kvp_last_error()
    side.synchronize()
    assert lib.kvp_attn_workspace_count() == n0, "the allocation-free entry made a workspace"
    assert lib.kvp_attn_forward_range(*args, ref.data_ptr(), nq, D, heads, key_begin, keys,
                                      stream) == 0, lib.kvp_last_error()
    side.synchronize()
    splits = api.attn_splits(dt, nq, heads, 1, keys - key_begin)
    if splits > 1:
        # one more buffer, unless the per-device bound of 8 evicted another
        assert lib.kvp_attn_workspace_count() == min(n0 + 1, max(n0, 8))
    n1 = lib.kvp_attn_workspace_count()
    assert lib.kvp_attn_workspace_release(stream) == 0
    assert lib.kvp_attn_workspace_count() == n1 - (1 if splits > 1 else 0)
    return got, ref, splits


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

#pragma once
// Internal helpers shared by the HIP translation units and the host C++ of
// libkvpersist.so. Not installed; the public surface is include/*.h.

#include <cstddef>

namespace kvp {

// Record a failure for kvp_last_error() (thread-local text).
void set_error(const char* fmt, ...);
void clear_error();

// Library stream for the reference-signature attention entry points.
void* library_stream();

// Core attention launch (attn_fwd.hip). Queries q[frame*q_fstride + row*D]
// for rows [0, nq) of `frames` frames; keys [key_begin, key_end) against
// k/v bases offset by frame*kv_fstride elements and kvmap offset by
// frame*map_fstride entries. dtype 0 = fp32, 1 = bf16. Returns 0 on success.
int launch_attention(int dtype, const void* q, const void* k, const void* v,
                     const void* arena, const long* kvmap, void* out, int nq,
                     int D, int heads, int frames, long q_fstride,
                     long kv_fstride, long map_fstride, long key_begin,
                     long key_end, void* stream);

int attention_splits(int dtype, int nq, int heads, int frames, long span);

}  // namespace kvp

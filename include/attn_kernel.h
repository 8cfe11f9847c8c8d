#pragma once

// KVMap-indirected multi-head attention (MI355X / gfx950 HIP kernels).
//
// out = softmax(Q K^T / sqrt(128)) V per head, online softmax over key
// tiles, fp32 accumulation. Key row j is read through an optional KVMap:
// KVMap[j] >= 0 -> arena row KVMap[j] (arena row = K row || V row, stride
// 2*D elements); KVMap[j] < 0 or KVMap == nullptr -> original K/V row j.
// Where a row is read from never changes the arithmetic, so outputs are
// bitwise identical across gating policies.
//
// Modes (reference: src/attn_kernel.h:6-29):
//   intra : frame f attends to its own T keys; Q/K/V/map pre-offset.
//   cross : causal temporal prefix, frame f attends to keys [0, (f+1)*T) of
//           the FULL K/V/map buffers; Q/Out pre-offset to the frame.
//
// The two functions below keep the reference declarations verbatim
// (C++ linkage, void return, async on the library stream — the null stream
// unless kvp_set_stream() changed it). Errors are recorded for
// kvp_last_error(); callers check with hipGetLastError / a sync, as the
// reference's callers did with CUDA. They forward to the C-ABI entry points
// of kvp_c_api.h, which also provides bf16 and sliding-window variants.

#include "kvp_c_api.h"

void attn_forward_launcher(const float* d_q, const float* d_k,
                           const float* d_v, const float* d_arena,
                           const long* d_kvmap, float* d_out,
                           int frames, int T, int D, int heads,
                           bool remap);

void attn_forward_single_frame(const float* d_q_f, const float* d_k,
                               const float* d_v, const float* d_arena,
                               const long* d_kvmap_f, float* d_out_f,
                               int T, int D, int heads, int cross,
                               int frame_idx);

// Tile constants of the reference API surface (reference:
// src/attn_kernel.h:31-32). The gfx950 kernels tile differently
// (kvp_attn_block_queries / kvp_attn_block_keys report their shapes); these
// stay exported so code that sized buffers with them still compiles.
static const int ATTENTION_KTILE = 64;
static const int ATTENTION_WARPS = 8;

#pragma once

/*
 * C-ABI of libkvpersist.so, upstream K/V producer: the random-init DiT
 * self-attention stack whose per-layer K/V the arena persists
 * (reference: src/backbone.py:8-67, src/config.py:6-27), gfx950 native.
 *
 * Conventions are those of kvp_c_api.h: device pointers owned by the caller,
 * int returns 0 = success with the text in kvp_last_error(), token-major
 * [rows, D] layout (rows = frames * tokens_per_frame), dtype 0 = fp32,
 * 1 = bf16 (raw uint16 bit patterns). Device pointers must be 16-byte
 * aligned. `stream` is a hipStream_t (NULL = null stream).
 *
 * The reference returns per-layer k, v as (b, heads, t, head_dim) views of
 * its qkv projection; its element (b, h, t, d) is element
 * (b*T + t, h*128 + d) of the token-major buffers written here, the layout
 * the attention entry points and the arena take.
 */

#include "kvp_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* nn.LayerNorm over the last dim (reference: src/backbone.py:28,48):
 * y = (x - mean) / sqrt(var + eps) * gamma + beta per row, fp32 statistics,
 * biased variance. gamma/beta fp32 [D]. D a multiple of 4, at most 4096. */
int kvp_layer_norm(int in_dtype, int out_dtype, const void* x,
                   const float* gamma, const float* beta, void* y, long rows,
                   int D, float eps, void* stream);

/* nn.Linear (reference: src/backbone.py:13-14,44):
 * y[rows, out] = x[rows, in] W[out, in]^T + bias (+ y when accumulate != 0,
 * fp32 output only). W has the storage dtype of x; bias fp32 [out] or NULL.
 * (in_dtype, out_dtype): (0, 0), (1, 1) or (1, 0). Any shape: bf16 shapes
 * with in % 64 == 0, out % 128 == 0 and 16-byte aligned operands run on the
 * grouped projection kernel (kvp_proj_gemm), every other shape and fp32 on
 * this library's generic fp32-matrix-core kernel; no library GEMM. */
int kvp_linear(int in_dtype, int out_dtype, const void* x, const void* w,
               const float* bias, void* y, long rows, int in_features,
               int out_features, int accumulate, void* stream);

/* Grouped bf16 projection on this library's gfx950 MFMA kernel: for
 * g < groups (1..3), out_g[r, n] = x[r, :] . w[g*N + n, :] + bias[g*N + n]
 * (+ out_g[r, n] when accumulate != 0). x [rows, K] and w [groups*N, K]
 * bf16, bias fp32 [groups*N] or NULL, out_g [rows, N] bf16 (out_dtype 1) or
 * fp32 (out_dtype 0, the only one that may accumulate). One launch serves
 * all groups: the q/k/v row blocks of qkv_proj written to three outputs, or
 * out_proj added into the fp32 residual stream (reference:
 * src/backbone.py:13-14,18-22,32-33). K a multiple of 64, N a multiple of
 * tile_n: 128 = 128 x 128 tiles, two workgroups per CU (the faster form at
 * the backbone's shapes); 256 = 256 x 256 tiles, one workgroup per CU.
 * Unused outputs may be NULL. */
int kvp_proj_gemm(const void* x, const void* w, const float* bias,
                  void* out0, void* out1, void* out2, int groups, long rows,
                  int K, int N, int out_dtype, int accumulate, int tile_n,
                  void* stream);

/* One block's LayerNorm + qkv_proj (reference: src/backbone.py:13,18-19,32):
 * xn = LN(x) (x fp32 residual stream [rows, D]), then q, k, v [rows, D] =
 * xn W_{q,k,v}^T + b_{q,k,v} with W = qkv_weight [3D, D] (rows 0..D-1 -> q,
 * D..2D-1 -> k, 2D..3D-1 -> v) and qkv_bias fp32 [3D]. xn is caller scratch
 * [rows, D] of the model dtype. */
int kvp_qkv_project(int dtype, const float* x, const float* ln_weight,
                    const float* ln_bias, const void* qkv_weight,
                    const float* qkv_bias, void* xn, void* q, void* k, void* v,
                    long rows, int D, void* stream);

/* SelfAttentionBackbone(cfg, init="random", seed) (reference:
 * src/backbone.py:36-56). hidden_dim must equal num_heads * 128. Parameters
 * are initialised on the device: Linear weights normal(0, 0.02), Linear
 * biases 0, LayerNorm weight 1 and bias 0; the normals come from this
 * library's own seeded generator (identical for equal seeds), not torch's.
 * The two projections of each block are stored in the model dtype, every
 * other parameter in fp32. Returns NULL on a bad config. An object runs one
 * forward at a time (its activation scratch is shared between calls and
 * grown, with a device synchronisation, when more frames arrive). */
void* kvp_backbone_create(int dtype, int num_layers, int tokens_per_frame,
                          int hidden_dim, int num_heads, int latent_channels,
                          unsigned long seed);
void kvp_backbone_destroy(void* bb);
/* sum(p.numel() for p in model.parameters()) (reference:
 * tests/test_skeleton.py:8-17,28-32). */
long kvp_backbone_param_count(void* bb);
/* Parameter tensors, named and ordered as the reference's state_dict
 * ("token_embed.weight", "blocks.<i>.norm.weight",
 * "blocks.<i>.attn.qkv_proj.weight", ..., "final_norm.bias"). */
int kvp_backbone_num_tensors(void* bb);
const char* kvp_backbone_tensor_name(void* bb, int index);
int kvp_backbone_param_info(void* bb, const char* name, void** dev_ptr,
                            long* numel, int* dtype);
/* Host fp32 in / out; bf16 parameters are rounded to nearest even on the
 * way in and widened on the way out. */
int kvp_backbone_set_param(void* bb, const char* name, const float* host,
                           long numel);
int kvp_backbone_get_param(void* bb, const char* name, float* host,
                           long numel);
/* SelfAttentionBackbone.forward (reference: src/backbone.py:58-67).
 * latents: fp32, frames * latent_channels * tokens_per_frame values per
 * call, each frame read as [tokens_per_frame, latent_channels] rows (the
 * reference's reshape of (b, C, rows, cols) latents, no permute).
 * hidden (fp32 [frames*T, D], may be NULL): final_norm output.
 * k_out, v_out (model dtype): layer l's K/V at element offset
 * l * layer_stride, each [frames*T, D]; q_out likewise or NULL.
 * layer_stride >= frames*T*D. */
int kvp_backbone_forward(void* bb, const float* latents, int frames,
                         float* hidden, void* q_out, void* k_out, void* v_out,
                         long layer_stride, void* stream);

#ifdef __cplusplus
}
#endif

// KVMap-indirected flash attention for MI355X (gfx950, CDNA4).
//
// Computes, per head h and query row q,
//     out[q, h] = softmax_j( Q[q,h] . K[j,h] / sqrt(128) ) V[j,h]
// over a key range [key_begin, key_end), reading key row j through the
// optional KVMap (reference semantics: src/gated_attention_kernel.cu:73-85
// and :118-130): map[j] >= 0 -> arena row map[j] = [K row | V row] with
// stride 2*D elements, otherwise the original K/V row j.
//
// Work decomposition (one launch):
//   workgroup = 4 waves x 32 query rows = 128 queries of one head, over one
//   key split; logical workgroup ids are (frame, head, split, q-block) with
//   q-block fastest, remapped so that each XCD receives a contiguous range
//   (hardware dispatches workgroups round-robin over the 8 XCDs), which keeps
//   the q-blocks sharing a key range on one L2.
//   When frames*heads*q-blocks would underfill the 256 CUs, the key range is
//   split and a combine kernel merges the per-split (O, logsumexp) partials.
//
// Per wave, per key tile (MFMA 32x32, fp32 accumulate):
//   S^T[key, q] = K[key, :] . Q[q, :]      A = K (LDS), B = Q (registers)
//   online softmax per query               lane owns one query column
//   O^T[d, q]  += V^T[d, key] P^T[key, q]   A = V^T (LDS), B = P^T (regs)
// Each lane holds one query (lane % 32) in every accumulator, so the softmax
// max/sum need one exchange between the two 32-lane halves only, and the
// output rescale is lane-local.
//
// bf16 path: v_mfma_f32_32x32x16_bf16; K tile [64][128] row-major and V tile
// transposed to [128][64] in LDS (16-byte chunks XOR-swizzled against bank
// conflicts); P is rounded to bf16 for the PV product.
// fp32 path: v_mfma_f32_32x32x2_f32; K and V tiles [32][128(+4 pad)] fp32.
//
// Invalid query rows (q >= nq) are clamped for loads and never stored; all
// threads reach every barrier. Invalid key rows of the last tile are zero in
// LDS and masked to -inf before the softmax.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <vector>

#include "kvp_c_api.h"
#include "kvp_internal.h"

namespace kvp {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

constexpr int kHeadDim = 128;
constexpr int kThreads = 256;
constexpr int kBlockQ = 128;  // 4 waves x 32 queries
constexpr int kNumXcd = 8;
constexpr float kLog2e = 1.4426950408889634f;

constexpr int kBf16BlockKeys = 64;
constexpr int kF32BlockKeys = 32;
constexpr int kF32RowPad = 4;  // floats of padding per LDS row (fp32 path)
constexpr int kF32LdsRow = kHeadDim + kF32RowPad;

struct AttnArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* arena;
    const long* kvmap;
    void* out;
    float* part_o;    // [splits][frames][nq][D] normalised partial O
    float* part_lse;  // [splits][frames][heads][nq] log2-sum-exp
    long q_fstride;   // elements between frames of q / out
    long kv_fstride;  // elements between frames of k / v
    long map_fstride; // entries between frames of kvmap
    long key_begin;
    long key_end;
    long keys_per_split;
    int nq;
    int D;
    int heads;
    int frames;
    int splits;
    int nqb;
    float scale_log2;  // log2(e) / sqrt(head_dim)
};

__device__ __forceinline__ int xcd_remap(int bid, int n) {
    const int per = n / kNumXcd;
    const int rem = n % kNumXcd;
    const int xcd = bid % kNumXcd;
    const int idx = bid / kNumXcd;
    return xcd < rem ? xcd * (per + 1) + idx
                     : rem * (per + 1) + (xcd - rem) * per + idx;
}

struct WgCoord {
    int qb, split, head, frame;
};

__device__ __forceinline__ WgCoord decode_wg(const AttnArgs& a) {
    int r = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    WgCoord c;
    c.qb = r % a.nqb;
    r /= a.nqb;
    c.split = r % a.splits;
    r /= a.splits;
    c.head = r % a.heads;
    c.frame = r / a.heads;
    return c;
}

// Value of x held by lane (lane ^ 32).
__device__ __forceinline__ float other_half(float x) {
    return __shfl_xor(x, 32);
}

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

// Writes the normalised result (or the split partial) of one wave.
// o[nb][v] holds O^T[d = 32*nb + 8*(v/4) + 4*hh + v%4][q].
template <typename OutT>
__device__ __forceinline__ void store_rows(const AttnArgs& a, const WgCoord& c,
                                           int q, int hh, const f32x16 (&o)[4],
                                           float m_run, float l_run) {
    if (q >= a.nq) return;
    const float inv_l = 1.0f / l_run;
    const int col0 = c.head * kHeadDim + 4 * hh;
    if (a.splits == 1) {
        OutT* out = reinterpret_cast<OutT*>(a.out) + (long)c.frame * a.q_fstride +
                    (long)q * a.D + col0;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * nb + 8 * g;
                if constexpr (sizeof(OutT) == 4) {
                    f32x4 w;
                    w[0] = o[nb][4 * g + 0] * inv_l;
                    w[1] = o[nb][4 * g + 1] * inv_l;
                    w[2] = o[nb][4 * g + 2] * inv_l;
                    w[3] = o[nb][4 * g + 3] * inv_l;
                    *reinterpret_cast<f32x4*>(out + d) = w;
                } else {
                    typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
                    bf16x4 w;
                    w[0] = (__bf16)(o[nb][4 * g + 0] * inv_l);
                    w[1] = (__bf16)(o[nb][4 * g + 1] * inv_l);
                    w[2] = (__bf16)(o[nb][4 * g + 2] * inv_l);
                    w[3] = (__bf16)(o[nb][4 * g + 3] * inv_l);
                    *reinterpret_cast<bf16x4*>(out + d) = w;
                }
            }
        }
    } else {
        const long slab = (long)c.split * a.frames + c.frame;
        float* po = a.part_o + (slab * a.nq + q) * (long)a.D + col0;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f32x4 w;
                w[0] = o[nb][4 * g + 0] * inv_l;
                w[1] = o[nb][4 * g + 1] * inv_l;
                w[2] = o[nb][4 * g + 2] * inv_l;
                w[3] = o[nb][4 * g + 3] * inv_l;
                *reinterpret_cast<f32x4*>(po + 32 * nb + 8 * g) = w;
            }
        }
        if (hh == 0) {
            a.part_lse[(slab * a.heads + c.head) * (long)a.nq + q] =
                m_run + __log2f(l_run);
        }
    }
}

// One online-softmax update for a lane's query over n fp32 scores held in
// s (already -inf where masked). Returns the correction factor for O.
template <int N>
__device__ __forceinline__ float softmax_update(float (&s)[N], float scale_log2,
                                                float& m_run, float& l_run) {
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < N; ++i) mx = fmaxf(mx, s[i]);
    mx = fmaxf(mx, other_half(mx));
    const float m_new = fmaxf(m_run, mx * scale_log2);
    const float corr = fast_exp2(m_run - m_new);
    float rs = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        s[i] = fast_exp2(fmaf(s[i], scale_log2, -m_new));
        rs += s[i];
    }
    rs += other_half(rs);
    l_run = l_run * corr + rs;
    m_run = m_new;
    return corr;
}

// ---------------------------------------------------------------------------
// bf16 kernel
// ---------------------------------------------------------------------------

constexpr int kBf16KBytes = kBf16BlockKeys * kHeadDim * 2;  // 16 KiB
constexpr int kBf16VBytes = kHeadDim * kBf16BlockKeys * 2;  // 16 KiB

template <typename OutT>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_bf16_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kBf16KBytes + kBf16VBytes];
    unsigned char* ks_lds = lds;
    unsigned char* vt_lds = lds + kBf16KBytes;

    const WgCoord c = decode_wg(a);
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int hh = lane >> 5;

    const long kbeg = a.key_begin + (long)c.split * a.keys_per_split;
    long kend = kbeg + a.keys_per_split;
    if (kend > a.key_end) kend = a.key_end;

    const __bf16* Q = reinterpret_cast<const __bf16*>(a.q) + (long)c.frame * a.q_fstride;
    const __bf16* K = reinterpret_cast<const __bf16*>(a.k) + (long)c.frame * a.kv_fstride;
    const __bf16* V = reinterpret_cast<const __bf16*>(a.v) + (long)c.frame * a.kv_fstride;
    const __bf16* A = reinterpret_cast<const __bf16*>(a.arena);
    const long* map = a.kvmap ? a.kvmap + (long)c.frame * a.map_fstride : nullptr;
    const int hoff = c.head * kHeadDim;
    const long D = a.D;

    // Query fragment (B operand of S^T = K Q^T): lane holds
    // Q[q][16*ks + 8*hh .. +8) for ks = 0..7.
    const int q = c.qb * kBlockQ + wave * 32 + lq;
    const int qc = q < a.nq ? q : a.nq - 1;
    bf16x8 qf[8];
    {
        const __bf16* qp = Q + (long)qc * D + hoff + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            qf[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qp + 16 * ks));
    }

    // Global->LDS staging assignment: 16-byte chunk ch of the head slice,
    // keys 4*grp .. 4*grp+3 of the tile.
    const int ld_ch = tid & 15;
    const int ld_grp = tid >> 4;

    u32x4 kr[4], vr[4];
    auto load_tile = [&](long t0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long j = t0 + 4 * ld_grp + i;
            if (j < kend) {
                const long m = map ? map[j] : -1L;
                const __bf16* kp = m >= 0 ? A + m * 2 * D + hoff : K + j * D + hoff;
                const __bf16* vp = m >= 0 ? A + m * 2 * D + D + hoff : V + j * D + hoff;
                kr[i] = *reinterpret_cast<const u32x4*>(kp + 8 * ld_ch);
                vr[i] = *reinterpret_cast<const u32x4*>(vp + 8 * ld_ch);
            } else {
                kr[i] = u32x4{0u, 0u, 0u, 0u};
                vr[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tile = [&]() {
        // K: row-major [64][256 B], chunk swizzle ch ^ (row & 15).
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * ld_grp + i;
            *reinterpret_cast<u32x4*>(ks_lds + row * 256 + ((ld_ch ^ (row & 15)) << 4)) = kr[i];
        }
        // V: transposed [128 d][64 keys]. Within each group of 16 keys the
        // position is 8*((k>>2)&1) + 4*(k>>3) + (k&3), so that lane half hh
        // of the PV MFMA reads its 8 keys as one contiguous 16-byte chunk.
        const int pos0 = 16 * (ld_grp >> 2) + 8 * (ld_grp & 1) + 4 * ((ld_grp >> 1) & 1);
        const int vch = pos0 >> 3;
        const int vsub = (pos0 & 7) << 1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const unsigned x0 = vr[0][e], x1 = vr[1][e], x2 = vr[2][e], x3 = vr[3][e];
            u32x2 lo, hi;
            lo[0] = (x0 & 0xffffu) | (x1 << 16);
            lo[1] = (x2 & 0xffffu) | (x3 << 16);
            hi[0] = (x0 >> 16) | (x1 & 0xffff0000u);
            hi[1] = (x2 >> 16) | (x3 & 0xffff0000u);
            const int d0 = 8 * ld_ch + 2 * e;
            const int d1 = d0 + 1;
            *reinterpret_cast<u32x2*>(vt_lds + d0 * 128 + ((vch ^ (d0 & 7)) << 4) + vsub) = lo;
            *reinterpret_cast<u32x2*>(vt_lds + d1 * 128 + ((vch ^ (d1 & 7)) << 4) + vsub) = hi;
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[nb][v] = 0.f;
    float m_run = -INFINITY;
    float l_run = 0.f;

    long t0 = kbeg;
    if (t0 < kend) load_tile(t0);
    for (; t0 < kend; t0 += kBf16BlockKeys) {
        store_tile();
        __syncthreads();
        if (t0 + kBf16BlockKeys < kend) load_tile(t0 + kBf16BlockKeys);

        // S^T for two 32-key blocks.
        f32x16 s0, s1;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            s0[v] = 0.f;
            s1[v] = 0.f;
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int chs = ((2 * ks + hh) ^ (lq & 15)) << 4;
            const bf16x8 ka = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(ks_lds + lq * 256 + chs));
            const bf16x8 kb = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(ks_lds + (32 + lq) * 256 + chs));
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[ks], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kb, qf[ks], s1, 0, 0, 0);
        }

        float s[32];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            s[v] = s0[v];
            s[16 + v] = s1[v];
        }
        if (t0 + kBf16BlockKeys > kend) {
            const long lim = kend - t0;
#pragma unroll
            for (int v = 0; v < 32; ++v) {
                const int key = 32 * (v >> 4) + 8 * ((v & 15) >> 2) + 4 * hh + (v & 3);
                if (key >= lim) s[v] = -INFINITY;
            }
        }
        const float corr = softmax_update<32>(s, a.scale_log2, m_run, l_run);

        bf16x8 pb[4];
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) pb[g][i] = (__bf16)s[8 * g + i];

#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
            for (int v = 0; v < 16; ++v) o[nb][v] *= corr;
            const int d = 32 * nb + lq;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int ch = 2 * g + hh;
                const bf16x8 va = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4*>(vt_lds + d * 128 + ((ch ^ (d & 7)) << 4)));
                o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[g], o[nb], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    store_rows<OutT>(a, c, q, hh, o, m_run, l_run);
}

// ---------------------------------------------------------------------------
// fp32 kernel
// ---------------------------------------------------------------------------

constexpr int kF32TileFloats = kF32BlockKeys * kF32LdsRow;

__global__ __launch_bounds__(kThreads, 2) void attn_fwd_f32_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float lds[2 * kF32TileFloats];
    float* ks_lds = lds;
    float* vs_lds = lds + kF32TileFloats;

    const WgCoord c = decode_wg(a);
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int hh = lane >> 5;

    const long kbeg = a.key_begin + (long)c.split * a.keys_per_split;
    long kend = kbeg + a.keys_per_split;
    if (kend > a.key_end) kend = a.key_end;

    const float* Q = reinterpret_cast<const float*>(a.q) + (long)c.frame * a.q_fstride;
    const float* K = reinterpret_cast<const float*>(a.k) + (long)c.frame * a.kv_fstride;
    const float* V = reinterpret_cast<const float*>(a.v) + (long)c.frame * a.kv_fstride;
    const float* A = reinterpret_cast<const float*>(a.arena);
    const long* map = a.kvmap ? a.kvmap + (long)c.frame * a.map_fstride : nullptr;
    const int hoff = c.head * kHeadDim;
    const long D = a.D;

    // Query fragment: lane holds Q[q][8*j + 4*hh .. +4) for j = 0..15;
    // MFMA k-step (j, i) pairs head dim 8*j + 4*hh + i of both operands.
    const int q = c.qb * kBlockQ + wave * 32 + lq;
    const int qc = q < a.nq ? q : a.nq - 1;
    f32x4 qf[16];
    {
        const float* qp = Q + (long)qc * D + hoff + 4 * hh;
#pragma unroll
        for (int j = 0; j < 16; ++j) qf[j] = *reinterpret_cast<const f32x4*>(qp + 8 * j);
    }

    // Staging: 16-byte chunk ch (4 floats) of the head slice, keys grp + 8*i.
    const int ld_ch = tid & 31;
    const int ld_grp = tid >> 5;

    f32x4 kr[4], vr[4];
    auto load_tile = [&](long t0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long j = t0 + ld_grp + 8 * i;
            if (j < kend) {
                const long m = map ? map[j] : -1L;
                const float* kp = m >= 0 ? A + m * 2 * D + hoff : K + j * D + hoff;
                const float* vp = m >= 0 ? A + m * 2 * D + D + hoff : V + j * D + hoff;
                kr[i] = *reinterpret_cast<const f32x4*>(kp + 4 * ld_ch);
                vr[i] = *reinterpret_cast<const f32x4*>(vp + 4 * ld_ch);
            } else {
                kr[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                vr[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = ld_grp + 8 * i;
            *reinterpret_cast<f32x4*>(ks_lds + row * kF32LdsRow + 4 * ld_ch) = kr[i];
            *reinterpret_cast<f32x4*>(vs_lds + row * kF32LdsRow + 4 * ld_ch) = vr[i];
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[nb][v] = 0.f;
    float m_run = -INFINITY;
    float l_run = 0.f;

    long t0 = kbeg;
    if (t0 < kend) load_tile(t0);
    for (; t0 < kend; t0 += kF32BlockKeys) {
        store_tile();
        __syncthreads();
        if (t0 + kF32BlockKeys < kend) load_tile(t0 + kF32BlockKeys);

        f32x16 st;
#pragma unroll
        for (int v = 0; v < 16; ++v) st[v] = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const f32x4 ka = *reinterpret_cast<const f32x4*>(ks_lds + lq * kF32LdsRow + 8 * j + 4 * hh);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[i], qf[j][i], st, 0, 0, 0);
        }

        float s[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) s[v] = st[v];
        if (t0 + kF32BlockKeys > kend) {
            const long lim = kend - t0;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int key = 8 * (v >> 2) + 4 * hh + (v & 3);
                if (key >= lim) s[v] = -INFINITY;
            }
        }
        const float corr = softmax_update<16>(s, a.scale_log2, m_run, l_run);

#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
            for (int v = 0; v < 16; ++v) o[nb][v] *= corr;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int key = 8 * (v >> 2) + 4 * hh + (v & 3);
                const float va = vs_lds[key * kF32LdsRow + 32 * nb + lq];
                o[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(va, s[v], o[nb], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    store_rows<float>(a, c, q, hh, o, m_run, l_run);
}

// ---------------------------------------------------------------------------
// split combine: out[q, h, :] = sum_s w_s O_s / sum_s w_s, w_s = 2^(lse_s - M)
// one thread per 4 output columns.
// ---------------------------------------------------------------------------
template <typename OutT>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int cols4 = a.D / 4;
    const long total = (long)a.frames * a.nq * cols4;
    if (gid >= total) return;
    const int c4 = (int)(gid % cols4);
    const long rq = gid / cols4;
    const int q = (int)(rq % a.nq);
    const int frame = (int)(rq / a.nq);
    const int head = (4 * c4) / kHeadDim;

    float mx = -INFINITY;
    for (int s = 0; s < a.splits; ++s) {
        const long slab = (long)s * a.frames + frame;
        mx = fmaxf(mx, a.part_lse[(slab * a.heads + head) * (long)a.nq + q]);
    }
    float wsum = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < a.splits; ++s) {
        const long slab = (long)s * a.frames + frame;
        const float w = fast_exp2(a.part_lse[(slab * a.heads + head) * (long)a.nq + q] - mx);
        const f32x4 po = *reinterpret_cast<const f32x4*>(a.part_o + (slab * a.nq + q) * (long)a.D + 4 * c4);
        wsum += w;
        acc[0] = fmaf(w, po[0], acc[0]);
        acc[1] = fmaf(w, po[1], acc[1]);
        acc[2] = fmaf(w, po[2], acc[2]);
        acc[3] = fmaf(w, po[3], acc[3]);
    }
    const float inv = 1.0f / wsum;
    OutT* out = reinterpret_cast<OutT*>(a.out) + (long)frame * a.q_fstride + (long)q * a.D + 4 * c4;
    if constexpr (sizeof(OutT) == 4) {
        f32x4 w = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        *reinterpret_cast<f32x4*>(out) = w;
    } else {
        typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
        bf16x4 w;
        w[0] = (__bf16)(acc[0] * inv);
        w[1] = (__bf16)(acc[1] * inv);
        w[2] = (__bf16)(acc[2] * inv);
        w[3] = (__bf16)(acc[3] * inv);
        *reinterpret_cast<bf16x4*>(out) = w;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

struct DeviceInfo {
    int cus = 256;
    int wg_per_cu_bf16 = 2;
    int wg_per_cu_f32 = 2;
    bool ok = false;
};

std::mutex g_mu;
std::vector<DeviceInfo> g_dev_info;
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::vector<Workspace> g_ws;

int current_device() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) return -1;
    return d;
}

DeviceInfo device_info(int dev) {
    std::lock_guard<std::mutex> lk(g_mu);
    if ((int)g_dev_info.size() <= dev) g_dev_info.resize(dev + 1);
    DeviceInfo& di = g_dev_info[dev];
    if (!di.ok) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) == hipSuccess) di.cus = prop.multiProcessorCount;
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, attn_fwd_bf16_kernel<__bf16>, kThreads, 0) == hipSuccess && nb > 0)
            di.wg_per_cu_bf16 = nb;
        nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, attn_fwd_f32_kernel, kThreads, 0) == hipSuccess && nb > 0)
            di.wg_per_cu_f32 = nb;
        di.ok = true;
    }
    return di;
}

void* workspace(int dev, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    Workspace& w = g_ws[dev];
    if (w.bytes < bytes) {
        // Growing waits for in-flight users of the old buffer.
        if (w.ptr) {
            (void)hipDeviceSynchronize();
            (void)hipFree(w.ptr);
            w.ptr = nullptr;
            w.bytes = 0;
        }
        size_t want = bytes + bytes / 4;
        if (hipMalloc(&w.ptr, want) != hipSuccess) {
            w.ptr = nullptr;
            return nullptr;
        }
        w.bytes = want;
    }
    return w.ptr;
}

// Estimated time in units of one key tile processed by a full wave of
// workgroups. Splitting divides the per-workgroup key loop but adds a
// combine pass whose cost grows with the number of splits.
int choose_splits(long base_wg, long ntiles, long slots) {
    if (slots <= 0) slots = 512;
    int best = 1;
    double best_t = 1e300;
    for (int s = 1; s <= 16; ++s) {
        if (s > 1 && ntiles / s < 4) break;
        const long wgs = base_wg * s;
        const long rounds = (wgs + slots - 1) / slots;
        const long per = (ntiles + s - 1) / s;
        double t = (double)rounds * (double)per;
        if (s > 1) t += 2.0 + 0.5 * (double)s * (double)base_wg / (double)slots;
        if (t < best_t - 1e-9) {
            best_t = t;
            best = s;
        }
    }
    return best;
}

struct LaunchPlan {
    int nqb, splits;
    long keys_per_split;
    long grid;
};

LaunchPlan plan_launch(int dtype, int nq, int heads, int frames, long span, const DeviceInfo& di) {
    LaunchPlan p;
    const int bk = dtype == 1 ? kBf16BlockKeys : kF32BlockKeys;
    p.nqb = (nq + kBlockQ - 1) / kBlockQ;
    const long base = (long)frames * heads * p.nqb;
    const long ntiles = (span + bk - 1) / bk;
    const long slots = (long)di.cus * (dtype == 1 ? di.wg_per_cu_bf16 : di.wg_per_cu_f32);
    int s = choose_splits(base, ntiles, slots);
    const long tiles_per = (ntiles + s - 1) / s;
    p.keys_per_split = tiles_per * bk;
    p.splits = (int)((span + p.keys_per_split - 1) / p.keys_per_split);
    p.grid = base * p.splits;
    return p;
}

}  // namespace

// Core launcher shared by all public attention entry points.
int launch_attention(int dtype, const void* q, const void* k, const void* v, const void* arena,
                     const long* kvmap, void* out, int nq, int D, int heads, int frames,
                     long q_fstride, long kv_fstride, long map_fstride, long key_begin,
                     long key_end, void* stream) {
    if (dtype != 0 && dtype != 1) {
        set_error("attention: dtype %d not supported (0 = fp32, 1 = bf16)", dtype);
        return 1;
    }
    if (heads <= 0 || D != heads * kHeadDim) {
        set_error("attention: head_dim must be 128 (D=%d heads=%d)", D, heads);
        return 1;
    }
    if (nq <= 0 || frames <= 0) {
        set_error("attention: empty launch (nq=%d frames=%d)", nq, frames);
        return 1;
    }
    if (key_end <= key_begin || key_begin < 0) {
        set_error("attention: empty or negative key range [%ld, %ld)", key_begin, key_end);
        return 1;
    }
    if (!q || !k || !v || !out) {
        set_error("attention: null q/k/v/out pointer");
        return 1;
    }
    if (kvmap && !arena) {
        set_error("attention: kvmap given without arena");
        return 1;
    }
    const int align = 16;
    if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out |
         (uintptr_t)arena) % align) {
        set_error("attention: q/k/v/out/arena must be 16-byte aligned");
        return 1;
    }
    const int dev = current_device();
    if (dev < 0) {
        set_error("attention: no HIP device available");
        return 1;
    }
    const DeviceInfo di = device_info(dev);
    const long span = key_end - key_begin;
    LaunchPlan p = plan_launch(dtype, nq, heads, frames, span, di);

    AttnArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.arena = arena;
    a.kvmap = kvmap;
    a.out = out;
    a.part_o = nullptr;
    a.part_lse = nullptr;
    a.q_fstride = q_fstride;
    a.kv_fstride = kv_fstride;
    a.map_fstride = map_fstride;
    a.key_begin = key_begin;
    a.key_end = key_end;
    a.keys_per_split = p.keys_per_split;
    a.nq = nq;
    a.D = D;
    a.heads = heads;
    a.frames = frames;
    a.splits = p.splits;
    a.nqb = p.nqb;
    a.scale_log2 = kLog2e / sqrtf((float)kHeadDim);

    if (p.splits > 1) {
        const size_t po = (size_t)p.splits * frames * nq * D * sizeof(float);
        const size_t pl = (size_t)p.splits * frames * heads * nq * sizeof(float);
        char* ws = static_cast<char*>(workspace(dev, po + pl + 256));
        if (!ws) {
            set_error("attention: workspace allocation of %zu bytes failed", po + pl);
            return 1;
        }
        a.part_o = reinterpret_cast<float*>(ws);
        a.part_lse = reinterpret_cast<float*>(ws + ((po + 255) / 256) * 256);
    }
    if (p.grid > 0x7fffffffL) {
        set_error("attention: grid too large");
        return 1;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == 1) {
        hipLaunchKernelGGL(attn_fwd_bf16_kernel<__bf16>, dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
    } else {
        hipLaunchKernelGGL(attn_fwd_f32_kernel, dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("attention launch: %s", hipGetErrorString(e));
        return 1;
    }
    if (p.splits > 1) {
        const long total = (long)frames * nq * (D / 4);
        const unsigned blocks = (unsigned)((total + 255) / 256);
        if (dtype == 1)
            hipLaunchKernelGGL(attn_combine_kernel<__bf16>, dim3(blocks), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL(attn_combine_kernel<float>, dim3(blocks), dim3(256), 0, st, a);
        e = hipGetLastError();
        if (e != hipSuccess) {
            set_error("attention combine launch: %s", hipGetErrorString(e));
            return 1;
        }
    }
    return 0;
}

int attention_splits(int dtype, int nq, int heads, int frames, long span) {
    if (nq <= 0 || heads <= 0 || frames <= 0 || span <= 0) return 0;
    DeviceInfo di;
    const int dev = current_device();
    if (dev >= 0) di = device_info(dev);
    return plan_launch(dtype, nq, heads, frames, span, di).splits;
}

}  // namespace kvp

extern "C" int kvp_attn_block_queries(int) { return kvp::kBlockQ; }
extern "C" int kvp_attn_block_keys(int dtype) {
    return dtype == 1 ? kvp::kBf16BlockKeys : kvp::kF32BlockKeys;
}
extern "C" int kvp_attn_splits(int dtype, int nq, int heads, int frames, long span) {
    return kvp::attention_splits(dtype, nq, heads, frames, span);
}

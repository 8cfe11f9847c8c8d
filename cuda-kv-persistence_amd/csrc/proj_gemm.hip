// Grouped bf16 projection GEMM for the K/V producer, gfx950 (CDNA4).
//
//   out_g[r, n] = sum_k x[r, k] * w[g*Ng + n, k] + bias[g*Ng + n]  (+ out_g[r, n])
//
// for groups g < G, with x [rows, K] and w [G*Ng, K] bf16 row-major (both
// K-contiguous), bias fp32, out_g [rows, Ng] bf16 or fp32 (fp32 may
// accumulate into itself: the residual add of out_proj). One launch covers
// every group, so the three q/k/v projections of a DiT block
// (reference: src/backbone.py:13,18-19) run as one grid written straight to
// three token-major outputs, and out_proj (src/backbone.py:22,32-33) adds
// into the fp32 residual stream in its epilogue.
//
// Two tilings share the operand layout below: the large-tile kernel (256 x
// 256, one workgroup per CU) and the small-tile kernel (128 x 128, two
// workgroups per CU, described at its definition), which is the faster one
// at the backbone's shapes and the one the q/k/v projection uses.
//
// Work decomposition (large tiles):
//   workgroup = 4 waves, output tile TN features x 256 tokens; wave (wn, wr)
//   owns (TN/2) x 128 of it as (TN/64) x 4 blocks of 32x32 accumulated by
//   v_mfma_f32_32x32x16_bf16 with A = w rows (features), B = x rows
//   (tokens): lane l holds token (l % 32) of a block and features
//   8*(v/4) + 4*(l/32) + v%4 in accumulator register v.
//   K advances in chunks of 64: both operand chunks ([TN][64] and [256][64]
//   bf16, 128-byte rows) arrive by buffer loads straight into a two-stage LDS
//   ring, 16-byte chunks XOR-swizzled by ((row >> 1) & 7) so that the
//   fragment reads (ds_read_b128, 16 rows per read phase) hit distinct banks.
//   Per k-step each wave reads its TN/64 + 4 fragments one step ahead of the
//   MFMAs; the next chunk's copies are all issued after the first k-step's
//   leading MFMAs, and the chunk barrier sits between the two halves of the
//   last k-step's MFMAs, so the next chunk's first fragment reads overlap
//   MFMAs.
//   The accumulators start at the bias. Epilogue: each wave stages its
//   outputs (converted to the output type) 32 tokens at a time in LDS as
//   token rows, then writes them (and, when accumulating, reads the
//   residual) as full 16-byte lanes along token rows, so global accesses are
//   row-contiguous.
//   Workgroups are numbered in bands of 4 token tiles x all feature tiles
//   (feature tile fastest within a band column) and remapped so that each XCD
//   receives a contiguous range: the workgroups resident on one XCD share a
//   few token tiles and a run of weight tiles through its L2.
//
// Token rows past `rows` read as zeros (buffer bounds) and are not stored.
// Requirements (checked on the host): K % 64 == 0, Ng % TN == 0, 16-byte
// aligned operands.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kvp_internal.h"

namespace kvp {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;

constexpr int kPThreads = 256;
constexpr int kPTileR = 256;   // tokens per workgroup tile (large-tile kernel)
constexpr int kPSmall = 128;   // features and tokens per tile (small-tile kernel)
constexpr int kPChunkK = 64;   // K per LDS stage
constexpr int kPRowBytes = kPChunkK * 2;
constexpr int kPBand = 4;      // token tiles per scheduling band
constexpr int kPNumXcd = 8;
constexpr int kPBufFlags = 0x00020000;

struct ProjArgs {
    const __bf16* x;
    const __bf16* w;
    const float* bias;
    void* out[3];
    long rows;
    int K;
    int Ng;
    int groups;
    int n_tiles;  // groups * Ng / TN
    int r_tiles;
};

#define PJ_LDS __attribute__((address_space(3)))

__device__ __forceinline__ void pj_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void pj_wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int OFF>
__device__ __forceinline__ u32x4 pj_lds_b128(unsigned addr) {
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF) : "memory");
    return r;
}

// Waits for every LDS read of the wave; the fragments are in/out operands so
// no use of them is scheduled before the wait.
template <int NF>
__device__ __forceinline__ void pj_lgkm_wait(u32x4 (&f)[NF]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < NF; ++i) asm volatile("" : "+v"(f[i]));
}

__device__ __forceinline__ int pj_xcd_remap(int bid, int n) {
    const int per = n / kPNumXcd;
    const int rem = n % kPNumXcd;
    const int xcd = bid % kPNumXcd;
    const int idx = bid / kPNumXcd;
    return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

template <int TN, typename OutT, bool kAcc>
__global__ __launch_bounds__(kPThreads, 1) void proj_gemm_bf16_kernel(ProjArgs a) {
    constexpr int JN = TN / 64;                 // 32-feature blocks per wave
    constexpr int kWBytes = TN * kPRowBytes;    // weight chunk bytes
    constexpr int kXBytes = kPTileR * kPRowBytes;
    constexpr int kWCopies = kWBytes / 1024 / 4;  // 1 KiB copies per wave per chunk
    constexpr int kXCopies = kXBytes / 1024 / 4;
    // stages: weights [2][kWBytes] then tokens [2][kXBytes]; the epilogue
    // reuses the space as per-wave output staging
    __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * (kWBytes + kXBytes)];
    auto w_stage = [&](int s) { return (unsigned)(uintptr_t)lds + (unsigned)(s * kWBytes); };
    auto x_stage = [&](int s) {
        return (unsigned)(uintptr_t)lds + (unsigned)(2 * kWBytes + s * kXBytes);
    };

    // ---- tile coordinates ----
    const int lid = pj_xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int band_tiles = kPBand * a.n_tiles;
    const int band = lid / band_tiles;
    const int in_band = lid % band_tiles;
    const int band_r0 = band * kPBand;
    int band_h = a.r_tiles - band_r0;
    if (band_h > kPBand) band_h = kPBand;
    const int rt = band_r0 + in_band % band_h;
    const int nt = in_band / band_h;
    const int tiles_per_group = a.Ng / TN;
    const int g = nt / tiles_per_group;
    const int n0 = (nt % tiles_per_group) * TN;  // feature offset within the group
    const long r0 = (long)rt * kPTileR;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int hh = lane >> 5;
    const int wn = wave & 1;
    const int wr = wave >> 1;

    // ---- copy setup: instruction i of a wave fills 1 KiB = 8 rows ----
    const unsigned kbytes = (unsigned)a.K * 2u;
    const __bf16* wg_base = a.w + ((long)g * a.Ng + n0) * a.K;
    const __bf16* xg_base = a.x + r0 * a.K;
    long xrows = a.rows - r0;
    if (xrows > kPTileR) xrows = kPTileR;
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__bf16*>(wg_base), (short)0, (int)(TN * kbytes), kPBufFlags);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__bf16*>(xg_base), (short)0, (int)(xrows * (long)kbytes), kPBufFlags);
    // rows of copy i: row = 8*(nwave_copies*wave + i) + lane/8; physical
    // chunk lane%8 holds logical chunk (lane%8) ^ ((row >> 1) & 7), and
    // (row >> 1) & 7 = (4*(i & 1) + lane/16) & 7 for every copy.
    const unsigned pch = (unsigned)(lane & 7);
    const unsigned lrow = (unsigned)(lane >> 3);
    const unsigned swz_even = (unsigned)((lane >> 4) & 7);
    const unsigned swz_odd = (unsigned)((4 + (lane >> 4)) & 7);
    const unsigned coff_even = 16u * (pch ^ swz_even);
    const unsigned coff_odd = 16u * (pch ^ swz_odd);

    auto issue_w = [&](int i, int stage, unsigned kofs) {
        const unsigned row = 8u * (unsigned)(kWCopies * wave + i) + lrow;
        const unsigned vo = row * kbytes + ((i & 1) ? coff_odd : coff_even);
        PJ_LDS void* d = (PJ_LDS void*)(uintptr_t)(unsigned)__builtin_amdgcn_readfirstlane(
            (int)(w_stage(stage) + 1024u * (unsigned)(kWCopies * wave + i)));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, d, 16, vo, (int)kofs, 0, 0);
    };
    auto issue_x = [&](int i, int stage, unsigned kofs) {
        const unsigned row = 8u * (unsigned)(kXCopies * wave + i) + lrow;
        const unsigned vo = row * kbytes + ((i & 1) ? coff_odd : coff_even);
        PJ_LDS void* d = (PJ_LDS void*)(uintptr_t)(unsigned)__builtin_amdgcn_readfirstlane(
            (int)(x_stage(stage) + 1024u * (unsigned)(kXCopies * wave + i)));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, d, 16, vo, (int)kofs, 0, 0);
    };
    // copy c of the chunk (0 .. kWCopies + kXCopies - 1), weights first
    auto issue_copy = [&](int c, int stage, unsigned kofs) {
        if (c < kWCopies)
            issue_w(c, stage, kofs);
        else
            issue_x(c - kWCopies, stage, kofs);
    };

    // ---- fragment addresses: row (lane % 32) of each 32-row block ----
    const unsigned fs = (unsigned)((lq >> 1) & 7);
    const unsigned w_row = (unsigned)(wn * (TN / 2) + lq) * kPRowBytes;
    const unsigned x_row = (unsigned)(wr * 128 + lq) * kPRowBytes;
    auto frag_off = [&](int ks) { return ((unsigned)(2 * ks + hh) ^ fs) << 4; };

    constexpr int NF = JN + 4;
    u32x4 fr[2][NF];
    auto read_frags = [&](u32x4 (&f)[NF], int stage, int ks) {
        const unsigned wa = w_stage(stage) + w_row + frag_off(ks);
        const unsigned xa = x_stage(stage) + x_row + frag_off(ks);
        f[0] = pj_lds_b128<0>(wa);
        if constexpr (JN > 1) f[1] = pj_lds_b128<32 * kPRowBytes>(wa);
        if constexpr (JN > 2) f[2] = pj_lds_b128<64 * kPRowBytes>(wa);
        if constexpr (JN > 3) f[3] = pj_lds_b128<96 * kPRowBytes>(wa);
        f[JN + 0] = pj_lds_b128<0>(xa);
        f[JN + 1] = pj_lds_b128<32 * kPRowBytes>(xa);
        f[JN + 2] = pj_lds_b128<64 * kPRowBytes>(xa);
        f[JN + 3] = pj_lds_b128<96 * kPRowBytes>(xa);
    };

    // Accumulators start at the bias: its loads overlap the prologue's copy
    // wait instead of stalling the epilogue.
    f32x16 acc[JN][4];
    {
        const float* bias = a.bias ? a.bias + (long)g * a.Ng + n0 + wn * (TN / 2) : nullptr;
#pragma unroll
        for (int i = 0; i < JN; ++i) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 b4 = bias ? *reinterpret_cast<const float4*>(bias + 32 * i + 8 * q4 +
                                                                          4 * hh)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j][4 * q4 + 0] = b4.x;
                    acc[i][j][4 * q4 + 1] = b4.y;
                    acc[i][j][4 * q4 + 2] = b4.z;
                    acc[i][j][4 * q4 + 3] = b4.w;
                }
            }
        }
    }

    auto mfma_half = [&](const u32x4 (&f)[NF], int half) {
#pragma unroll
        for (int i = 0; i < JN; ++i)
#pragma unroll
            for (int j = 2 * half; j < 2 * half + 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8, f[i]), __builtin_bit_cast(bf16x8, f[JN + j]),
                    acc[i][j], 0, 0, 0);
    };

    const int nk = a.K / kPChunkK;
    constexpr int kCopies = kWCopies + kXCopies;

    // prologue: chunk 0 into stage 0, its first fragments
#pragma unroll
    for (int c = 0; c < kCopies; ++c) issue_copy(c, 0, 0u);
    pj_wait_vm0();
    pj_barrier();
    read_frags(fr[0], 0, 0);

    for (int t = 0; t < nk; ++t) {
        const int st = t & 1;
        const bool more = t + 1 < nk;
        const unsigned knext = (unsigned)(t + 1) * kPRowBytes;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4 (&cur)[NF] = fr[ks & 1];
            u32x4 (&nxt)[NF] = fr[(ks + 1) & 1];
            pj_lgkm_wait(cur);
            if (ks < 3) read_frags(nxt, st, ks + 1);
            __builtin_amdgcn_s_setprio(1);
            mfma_half(cur, 0);
            __builtin_amdgcn_s_setprio(0);
            if (ks == 3 && more) {
                // chunk t+1 has landed for every wave once all pass here; all
                // reads of chunk t are complete (waited above)
                pj_wait_vm0();
                pj_barrier();
                read_frags(nxt, st ^ 1, 0);
            }
            if (ks == 0 && more) {
                // all of the next chunk's copies at once, as early as the ring
                // allows: their latency, not their issue, is what stalls
#pragma unroll
                for (int c = 0; c < kCopies; ++c) issue_copy(c, st ^ 1, knext);
            }
            __builtin_amdgcn_s_setprio(1);
            mfma_half(cur, 1);
            __builtin_amdgcn_s_setprio(0);
        }
    }

    // ---- epilogue: stage as token rows in LDS, row-contiguous store ----
    constexpr int kFeat = TN / 2;                   // features per wave
    constexpr int kEs = (int)sizeof(OutT);
    constexpr int kRowB = kFeat * kEs + 16;         // padded staging row (bytes)
    constexpr int kChunks = kFeat * kEs / 16;       // 16-byte chunks per row
    constexpr int kRowsPerPass = 64 / kChunks;      // rows one wave instruction covers
    static_assert(4 * 32 * kRowB <= 2 * (kWBytes + kXBytes), "staging exceeds LDS");
    pj_barrier();  // every wave has finished reading the operand stages
    OutT* out = static_cast<OutT*>(a.out[g]);
    unsigned char* sbase = lds + wave * 32 * kRowB;
    const int rchunk = lane % kChunks;
    const int rrow = lane / kChunks;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        unsigned char* wrow = sbase + lq * kRowB;
#pragma unroll
        for (int i = 0; i < JN; ++i) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float v0 = acc[i][j][4 * q4 + 0];
                const float v1 = acc[i][j][4 * q4 + 1];
                const float v2 = acc[i][j][4 * q4 + 2];
                const float v3 = acc[i][j][4 * q4 + 3];
                OutT* p = reinterpret_cast<OutT*>(wrow) + 32 * i + 8 * q4 + 4 * hh;
                if constexpr (kEs == 4) {
                    *reinterpret_cast<float4*>(p) = make_float4(v0, v1, v2, v3);
                } else {
                    struct alignas(8) B4 {
                        __bf16 v[4];
                    } o;
                    o.v[0] = (__bf16)v0;
                    o.v[1] = (__bf16)v1;
                    o.v[2] = (__bf16)v2;
                    o.v[3] = (__bf16)v3;
                    *reinterpret_cast<B4*>(p) = o;
                }
            }
        }
        // same-wave LDS accesses complete in order: the rows written above
        // are read back below, and the next block's writes follow these reads
#pragma unroll
        for (int pass = 0; pass < 32 / kRowsPerPass; ++pass) {
            const int row = pass * kRowsPerPass + rrow;
            const long r = r0 + wr * 128 + 32 * j + row;
            const u32x4 vals = *reinterpret_cast<const u32x4*>(sbase + row * kRowB + 16 * rchunk);
            if (r >= a.rows) continue;
            unsigned char* gp = reinterpret_cast<unsigned char*>(out + r * a.Ng + n0 + wn * kFeat) +
                                16 * rchunk;
            if constexpr (kAcc) {
                float4 y = *reinterpret_cast<const float4*>(gp);
                y.x += __uint_as_float(vals[0]);
                y.y += __uint_as_float(vals[1]);
                y.z += __uint_as_float(vals[2]);
                y.w += __uint_as_float(vals[3]);
                *reinterpret_cast<float4*>(gp) = y;
            } else {
                *reinterpret_cast<u32x4*>(gp) = vals;
            }
        }
    }
}

// Small-tile form: TN features x TR tokens per workgroup (128 x 128), two
// workgroups per CU (64 KiB of LDS each: K chunks of 64 in a two-stage ring,
// the same 128-byte swizzled rows as above); wave (wn, wr) owns (TN/2) x
// (TR/2) as (TN/64) x (TR/64) blocks. Each chunk's copies are issued right
// after the barrier that frees their stage. With two resident workgroups the
// one in its epilogue or waiting on copies leaves the MFMA pipe to the other,
// and four times as many tiles even out the rounds over the CUs.
template <int TN, int TR, typename OutT, bool kAcc>
__global__ __launch_bounds__(kPThreads, 2) void proj_gemm_bf16_small_kernel(ProjArgs a) {
    constexpr int JN = TN / 64, JR = TR / 64;
    constexpr int kWB = TN * kPRowBytes, kXB = TR * kPRowBytes, kSB = kWB + kXB;
    constexpr int kWC = kWB / 4096, kXC = kXB / 4096, kCP = kWC + kXC;  // copies per wave
    __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * kSB];

    const int lid = pj_xcd_remap((int)blockIdx.x, (int)gridDim.x);
    const int band_tiles = kPBand * a.n_tiles;
    const int band = lid / band_tiles;
    const int in_band = lid % band_tiles;
    const int band_r0 = band * kPBand;
    int band_h = a.r_tiles - band_r0;
    if (band_h > kPBand) band_h = kPBand;
    const int rt = band_r0 + in_band % band_h;
    const int nt = in_band / band_h;
    const int tiles_per_group = a.Ng / TN;
    const int g = nt / tiles_per_group;
    const int n0 = (nt % tiles_per_group) * TN;
    const long r0 = (long)rt * TR;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int hh = lane >> 5;
    const int wn = wave & 1;
    const int wr = wave >> 1;

    const unsigned kbytes = (unsigned)a.K * 2u;
    long xrows = a.rows - r0;
    if (xrows > TR) xrows = TR;
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__bf16*>(a.w + ((long)g * a.Ng + n0) * a.K), (short)0, (int)(TN * kbytes),
        kPBufFlags);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__bf16*>(a.x + r0 * a.K), (short)0, (int)(xrows * (long)kbytes), kPBufFlags);
    const unsigned lds0 = (unsigned)(uintptr_t)lds;
    // copy c of a chunk: 1 KiB block blk of the weight (c < kWC) or token
    // operand, rows 8*blk + lane/8, physical chunk lane % 8
    auto issue_copy = [&](int c, int stage, unsigned kofs) {
        const bool isw = c < kWC;
        const int blk = (isw ? kWC : kXC) * wave + (isw ? c : c - kWC);
        const unsigned row = 8u * (unsigned)blk + (unsigned)(lane >> 3);
        const unsigned lc = (unsigned)(lane & 7) ^ ((row >> 1) & 7u);
        const unsigned dst = lds0 + (unsigned)(stage * kSB) + (isw ? 0u : (unsigned)kWB) +
                             1024u * (unsigned)blk;
        PJ_LDS void* d = (PJ_LDS void*)(uintptr_t)(unsigned)__builtin_amdgcn_readfirstlane((int)dst);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(isw ? wrs : xrs, d, 16, row * kbytes + 16u * lc,
                                                 (int)kofs, 0, 0);
    };
    const unsigned fs = (unsigned)((lq >> 1) & 7);
    const unsigned w_row = (unsigned)(wn * (TN / 2) + lq) * kPRowBytes;
    const unsigned x_row = (unsigned)(wr * (TR / 2) + lq) * kPRowBytes;
    constexpr int NF = JN + JR;
    auto read_frags = [&](u32x4 (&f)[NF], int stage, int ks) {
        const unsigned fo = ((unsigned)(2 * ks + hh) ^ fs) << 4;
        const unsigned wa = lds0 + (unsigned)(stage * kSB) + w_row + fo;
        const unsigned xa = lds0 + (unsigned)(stage * kSB + kWB) + x_row + fo;
        f[0] = pj_lds_b128<0>(wa);
        if constexpr (JN > 1) f[1] = pj_lds_b128<32 * kPRowBytes>(wa);
        f[JN] = pj_lds_b128<0>(xa);
        if constexpr (JR > 1) f[JN + 1] = pj_lds_b128<32 * kPRowBytes>(xa);
    };
    static_assert(JN <= 2 && JR <= 2, "fragment reads cover two blocks per operand");

    f32x16 acc[JN][JR];
    {
        const float* bias = a.bias ? a.bias + (long)g * a.Ng + n0 + wn * (TN / 2) : nullptr;
#pragma unroll
        for (int i = 0; i < JN; ++i) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 b4 = bias ? *reinterpret_cast<const float4*>(bias + 32 * i + 8 * q4 +
                                                                          4 * hh)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int j = 0; j < JR; ++j) {
                    acc[i][j][4 * q4 + 0] = b4.x;
                    acc[i][j][4 * q4 + 1] = b4.y;
                    acc[i][j][4 * q4 + 2] = b4.z;
                    acc[i][j][4 * q4 + 3] = b4.w;
                }
            }
        }
    }

    const int nk = a.K / kPChunkK;
    constexpr int kFeat = TN / 2;
    constexpr int kEs = (int)sizeof(OutT);
    constexpr int kChunks = kFeat * kEs / 16;
    constexpr int kRowsPerPass = 64 / kChunks;
    constexpr int kPasses = 32 / kRowsPerPass;
    OutT* out = static_cast<OutT*>(a.out[g]);
    const int rchunk = lane % kChunks;
    const int rrow = lane / kChunks;
    // Accumulating (out_proj into the fp32 residual stream): every residual
    // value the wave adds in the epilogue, loaded all at once during the last
    // chunk's MFMAs (issued after the copies of that chunk, one chunk ahead),
    // so that their memory latency is not paid at the end of every tile.
    float4 resid[kAcc ? JR : 1][kAcc ? kPasses : 1];
    auto load_resid = [&]() {
#pragma unroll
        for (int j = 0; j < JR; ++j) {
#pragma unroll
            for (int pass = 0; pass < kPasses; ++pass) {
                const long r = r0 + wr * (TR / 2) + 32 * j + pass * kRowsPerPass + rrow;
                // every lane loads (a row past the end reads the last row; the
                // epilogue never writes such rows), so the loop's wait below
                // counts exactly these JR * kPasses loads
                const long rc = r < a.rows ? r : a.rows - 1;
                const float* gp = reinterpret_cast<const float*>(out) + rc * a.Ng + n0 +
                                  wn * kFeat + 4 * rchunk;
                resid[j][pass] = *reinterpret_cast<const float4*>(gp);
            }
        }
    };
#pragma unroll
    for (int c = 0; c < kCP; ++c) issue_copy(c, 0, 0u);
    u32x4 fr[2][NF];
    for (int t = 0; t < nk; ++t) {
        const int st = t & 1;
        // chunk t has landed for every wave after the barrier, and every
        // wave has finished chunk t-1, whose stage the next copies refill.
        // Before the last chunk, the only loads issued after chunk t's copies
        // are the residual loads (a wave's vector-memory operations complete
        // in issue order), which may stay in flight.
        if (kAcc && t == nk - 1 && nk >= 2)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(JR * kPasses) : "memory");
        else
            pj_wait_vm0();
        pj_barrier();
        if (t + 1 < nk) {
#pragma unroll
            for (int c = 0; c < kCP; ++c) issue_copy(c, st ^ 1, (unsigned)(t + 1) * kPRowBytes);
        }
        if constexpr (kAcc) {
            if (t == nk - 2) {
                asm volatile("" ::: "memory");  // the loads go out after the copies
                load_resid();
            }
        }
        read_frags(fr[0], st, 0);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4 (&cur)[NF] = fr[ks & 1];
            pj_lgkm_wait(cur);
            if (ks < 3) read_frags(fr[(ks + 1) & 1], st, ks + 1);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int i = 0; i < JN; ++i)
#pragma unroll
                for (int j = 0; j < JR; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, cur[i]), __builtin_bit_cast(bf16x8, cur[JN + j]),
                        acc[i][j], 0, 0, 0);
            __builtin_amdgcn_s_setprio(0);
        }
    }

    // epilogue: as in the large-tile kernel, 32 tokens at a time
    constexpr int kRowB = kFeat * kEs + 16;
    static_assert(4 * 32 * kRowB <= 2 * kSB, "staging exceeds LDS");
    if constexpr (kAcc) {
        if (nk < 2) load_resid();  // a one-chunk K: no earlier chunk to load under
    }
    pj_barrier();
    unsigned char* sbase = lds + wave * 32 * kRowB;
#pragma unroll
    for (int j = 0; j < JR; ++j) {
        unsigned char* wrow = sbase + lq * kRowB;
#pragma unroll
        for (int i = 0; i < JN; ++i) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float v0 = acc[i][j][4 * q4 + 0];
                const float v1 = acc[i][j][4 * q4 + 1];
                const float v2 = acc[i][j][4 * q4 + 2];
                const float v3 = acc[i][j][4 * q4 + 3];
                OutT* p = reinterpret_cast<OutT*>(wrow) + 32 * i + 8 * q4 + 4 * hh;
                if constexpr (kEs == 4) {
                    *reinterpret_cast<float4*>(p) = make_float4(v0, v1, v2, v3);
                } else {
                    struct alignas(8) B4 {
                        __bf16 v[4];
                    } o;
                    o.v[0] = (__bf16)v0;
                    o.v[1] = (__bf16)v1;
                    o.v[2] = (__bf16)v2;
                    o.v[3] = (__bf16)v3;
                    *reinterpret_cast<B4*>(p) = o;
                }
            }
        }
#pragma unroll
        for (int pass = 0; pass < 32 / kRowsPerPass; ++pass) {
            const int row = pass * kRowsPerPass + rrow;
            const long r = r0 + wr * (TR / 2) + 32 * j + row;
            const u32x4 vals = *reinterpret_cast<const u32x4*>(sbase + row * kRowB + 16 * rchunk);
            if (r >= a.rows) continue;
            unsigned char* gp = reinterpret_cast<unsigned char*>(out + r * a.Ng + n0 + wn * kFeat) +
                                16 * rchunk;
            if constexpr (kAcc) {
                float4 y = resid[j][pass];
                y.x += __uint_as_float(vals[0]);
                y.y += __uint_as_float(vals[1]);
                y.z += __uint_as_float(vals[2]);
                y.w += __uint_as_float(vals[3]);
                *reinterpret_cast<float4*>(gp) = y;
            } else {
                *reinterpret_cast<u32x4*>(gp) = vals;
            }
        }
    }
}

template <typename OutT, bool kAcc>
void launch_large(const ProjArgs& a, hipStream_t st) {
    const int grid = a.n_tiles * a.r_tiles;
    hipLaunchKernelGGL((proj_gemm_bf16_kernel<256, OutT, kAcc>), dim3((unsigned)grid),
                       dim3(kPThreads), 0, st, a);
}

template <typename OutT, bool kAcc>
void launch_small(const ProjArgs& a, hipStream_t st) {
    const int grid = a.n_tiles * a.r_tiles;
    hipLaunchKernelGGL((proj_gemm_bf16_small_kernel<kPSmall, kPSmall, OutT, kAcc>),
                       dim3((unsigned)grid), dim3(kPThreads), 0, st, a);
}


// ---------------------------------------------------------------------------
// Generic linear layer (shapes the grouped kernel does not tile, and fp32):
//
//   y[r, n] = sum_k x[r, k] * w[n, k] + bias[n]  (+ y[r, n])
//
// x [rows, K], w [N, K] row-major (K-contiguous), fp32 or bf16 (widened to
// fp32 in LDS), bias fp32 or null, y fp32 or bf16 (fp32 may accumulate into
// itself). fp32 matrix cores: v_mfma_f32_32x32x2_f32 (full fp32 products,
// fp32 accumulation). Workgroup = 4 waves, output tile 64 features x 64
// rows, wave (w & 1, w >> 1) owns 32 x 32 of it: lane l holds row (l % 32)
// of the block and features 8*(v/4) + 4*(l/32) + v%4 in accumulator v (A =
// w rows, B = x rows, as in the grouped kernel). K advances in chunks of 32;
// each chunk of w and x is staged in LDS as 64 rows of 32 values padded to
// 33, so that the 32 lanes of a half-wave reading one k of 32 rows hit 32
// distinct banks. Every global access is bounds-checked: any rows, K and N.
// The epilogue stages the 64 x 64 tile in the same LDS as rows (pitch 65)
// and stores it row by row, 16 lanes per 64-value row, 4 consecutive values
// per lane (one 16-byte fp32 / 8-byte bf16 store where the row and its
// alignment allow, per-value stores at ragged edges): a row's 256 bytes go
// out together instead of 4-byte pieces of 32 rows per instruction.
// ---------------------------------------------------------------------------
constexpr int kGTile = 64;
constexpr int kGChunk = 32;
constexpr int kGPitch = kGChunk + 1;
constexpr int kGOutPitch = kGTile + 1;
static_assert(kGTile * kGOutPitch <= 2 * kGTile * kGPitch, "output staging exceeds LDS");

struct GenericArgs {
    const void* x;
    const void* w;
    const float* bias;
    void* y;
    long rows;
    int K, N;
    int n_tiles;
};

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
    return (float)v;
}

template <typename InT, typename OutT, bool kAcc>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GenericArgs a) {
    __shared__ float lds[2 * kGTile * kGPitch];
    float* ws = lds;
    float* xs = lds + kGTile * kGPitch;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const long n0 = (long)(blockIdx.x % a.n_tiles) * kGTile;
    const long r0 = (long)(blockIdx.x / a.n_tiles) * kGTile;
    const InT* W = static_cast<const InT*>(a.w);
    const InT* X = static_cast<const InT*>(a.x);
    const int bn = 32 * (wave & 1);   // the wave's feature block within the tile
    const int br = 32 * (wave >> 1);  // its row block
    const int lr = lane & 31;
    const int lk = lane >> 5;
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
    for (int k0 = 0; k0 < a.K; k0 += kGChunk) {
        // 64 rows x 32 k of each operand: element e = tid + 256 j is row
        // e / 32, k e % 32 (a warp's consecutive lanes read consecutive k)
#pragma unroll
        for (int j = 0; j < kGTile * kGChunk / 256; ++j) {
            const int e = tid + 256 * j;
            const int row = e / kGChunk;
            const int kk = e % kGChunk;
            const long gk = (long)k0 + kk;
            const long gn = n0 + row;
            const long gr = r0 + row;
            ws[row * kGPitch + kk] = gn < a.N && gk < a.K ? to_f32(W[gn * a.K + gk]) : 0.f;
            xs[row * kGPitch + kk] = gr < a.rows && gk < a.K ? to_f32(X[gr * a.K + gk]) : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGChunk; kk += 2) {
            const float av = ws[(bn + lr) * kGPitch + kk + lk];
            const float bv = xs[(br + lr) * kGPitch + kk + lk];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    // stage: row br + lr of the tile, columns bn + 8*(v/4) + 4*lk + v%4
    // (the loop's last barrier has freed the operand tiles)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int col = bn + 8 * (v / 4) + 4 * lk + v % 4;
        const long n = n0 + col;
        lds[(br + lr) * kGOutPitch + col] = acc[v] + (a.bias && n < a.N ? a.bias[n] : 0.f);
    }
    __syncthreads();
    // 64 rows x 16 four-value groups, 4 per thread; 16 consecutive threads
    // cover one row
    const bool vec_ok = (a.N % 4) == 0 &&
                        ((uintptr_t)a.y % (4 * sizeof(OutT))) == 0;
#pragma unroll
    for (int j = 0; j < kGTile * kGTile / 4 / 256; ++j) {
        const int c = tid + 256 * j;
        const int row = c / (kGTile / 4);
        const int col = 4 * (c % (kGTile / 4));
        const long r = r0 + row;
        const long n = n0 + col;
        if (r >= a.rows || n >= a.N) continue;
        const float* src = lds + row * kGOutPitch + col;
        OutT* Y = static_cast<OutT*>(a.y) + r * a.N + n;
        if (vec_ok) {
            // n + 3 < N: N and n are multiples of 4
            float v4[4] = {src[0], src[1], src[2], src[3]};
            if constexpr (sizeof(OutT) == 4) {
                if constexpr (kAcc) {
                    const float4 y = *reinterpret_cast<const float4*>(Y);
                    v4[0] += y.x;
                    v4[1] += y.y;
                    v4[2] += y.z;
                    v4[3] += y.w;
                }
                *reinterpret_cast<float4*>(Y) = make_float4(v4[0], v4[1], v4[2], v4[3]);
            } else {
                struct alignas(8) B4 {
                    OutT v[4];
                } o;
#pragma unroll
                for (int i = 0; i < 4; ++i) o.v[i] = (OutT)v4[i];
                *reinterpret_cast<B4*>(Y) = o;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (n + i >= a.N) break;
                float val = src[i];
                if constexpr (kAcc) val += to_f32(Y[i]);
                Y[i] = (OutT)val;
            }
        }
    }
}

template <typename InT, typename OutT, bool kAcc>
void launch_generic(const GenericArgs& a, long grid, hipStream_t st) {
    hipLaunchKernelGGL((gemm_generic_kernel<InT, OutT, kAcc>), dim3((unsigned)grid), dim3(256), 0,
                       st, a);
}

}  // namespace

int launch_gemm_generic(int in_dtype, int out_dtype, const void* x, const void* w,
                        const float* bias, void* y, long rows, int K, int N, bool accumulate,
                        void* stream) {
    if (!((in_dtype == 0 && out_dtype == 0) || (in_dtype == 1 && (out_dtype == 0 || out_dtype == 1)))) {
        set_error("linear: dtype pair (%d, %d) not supported (fp32->fp32, bf16->bf16, "
                  "bf16->fp32)",
                  in_dtype, out_dtype);
        return 1;
    }
    if (rows <= 0 || K <= 0 || N <= 0) {
        set_error("linear: empty shape rows=%ld in=%d out=%d", rows, K, N);
        return 1;
    }
    if (accumulate && out_dtype != 0) {
        set_error("linear: accumulate needs fp32 output");
        return 1;
    }
    if (!x || !w || !y) {
        set_error("linear: null x/w/y pointer");
        return 1;
    }
    GenericArgs a;
    a.x = x;
    a.w = w;
    a.bias = bias;
    a.y = y;
    a.rows = rows;
    a.K = K;
    a.N = N;
    const long n_tiles = ((long)N + kGTile - 1) / kGTile;
    const long r_tiles = (rows + kGTile - 1) / kGTile;
    if (n_tiles * r_tiles > 0x7fffffffL) {
        set_error("linear: grid too large");
        return 1;
    }
    a.n_tiles = (int)n_tiles;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const long grid = n_tiles * r_tiles;
    if (in_dtype == 0) {
        if (accumulate)
            launch_generic<float, float, true>(a, grid, st);
        else
            launch_generic<float, float, false>(a, grid, st);
    } else if (out_dtype == 1) {
        launch_generic<__bf16, __bf16, false>(a, grid, st);
    } else if (accumulate) {
        launch_generic<__bf16, float, true>(a, grid, st);
    } else {
        launch_generic<__bf16, float, false>(a, grid, st);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("linear launch: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

namespace {
}  // namespace

int launch_proj_gemm(const void* x, const void* w, const float* bias, void* const* outs,
                     int groups, long rows, int K, int Ng, int out_dtype, bool accumulate,
                     int tile_n, void* stream) {
    if (groups < 1 || groups > 3 || rows <= 0 || K <= 0 || Ng <= 0) {
        set_error("proj_gemm: bad shape groups=%d rows=%ld K=%d N=%d", groups, rows, K, Ng);
        return 1;
    }
    if (tile_n != 128 && tile_n != 256) {
        set_error("proj_gemm: tile_n must be 128 or 256");
        return 1;
    }
    if (K % kPChunkK || Ng % tile_n || (long)K * 2 * kPTileR > 0x7fffffffL) {
        set_error("proj_gemm: shape K=%d N=%d not supported (K %% 64, N %% %d)", K, Ng, tile_n);
        return 2;
    }
    if (accumulate && out_dtype != 0) {
        set_error("proj_gemm: accumulate needs fp32 output");
        return 1;
    }
    if (!x || !w) {
        set_error("proj_gemm: null operand");
        return 1;
    }
    uintptr_t al = (uintptr_t)x | (uintptr_t)w | (uintptr_t)bias;
    for (int g = 0; g < groups; ++g) {
        if (!outs[g]) {
            set_error("proj_gemm: null output %d", g);
            return 1;
        }
        al |= (uintptr_t)outs[g];
    }
    if (al & 15u) {
        set_error("proj_gemm: operands must be 16-byte aligned");
        return 1;
    }
    const long tile_r = tile_n == 256 ? kPTileR : kPSmall;
    const long r_tiles = (rows + tile_r - 1) / tile_r;
    const long n_tiles = (long)groups * (Ng / tile_n);
    if (r_tiles * n_tiles > 0x7fffffffL) {
        set_error("proj_gemm: grid too large");
        return 1;
    }
    ProjArgs a;
    a.x = static_cast<const __bf16*>(x);
    a.w = static_cast<const __bf16*>(w);
    a.bias = bias;
    for (int g = 0; g < 3; ++g) a.out[g] = g < groups ? outs[g] : nullptr;
    a.rows = rows;
    a.K = K;
    a.Ng = Ng;
    a.groups = groups;
    a.n_tiles = (int)n_tiles;
    a.r_tiles = (int)r_tiles;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (tile_n == 256) {
        if (out_dtype == 1)
            launch_large<__bf16, false>(a, st);
        else if (accumulate)
            launch_large<float, true>(a, st);
        else
            launch_large<float, false>(a, st);
    } else {
        if (out_dtype == 1)
            launch_small<__bf16, false>(a, st);
        else if (accumulate)
            launch_small<float, true>(a, st);
        else
            launch_small<float, false>(a, st);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("proj_gemm launch: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

}  // namespace kvp

extern "C" int kvp_proj_gemm(const void* x, const void* w, const float* bias, void* out0,
                             void* out1, void* out2, int groups, long rows, int K, int N,
                             int out_dtype, int accumulate, int tile_n, void* stream) {
    void* outs[3] = {out0, out1, out2};
    const int rc = kvp::launch_proj_gemm(x, w, bias, outs, groups, rows, K, N, out_dtype,
                                         accumulate != 0, tile_n, stream);
    return rc == 0 ? 0 : 1;
}

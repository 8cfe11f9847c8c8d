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
// fp32 path: v_mfma_f32_32x32x2_f32; K and V tiles [32][128] fp32, 16-byte
// chunks XOR-swizzled in LDS, P kept in fp32.
//
// Invalid query rows (q >= nq) are clamped for loads and never stored; all
// threads reach every barrier. Invalid key rows of the last tile are zero in
// LDS and masked to -inf before the softmax.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <thread>
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

struct AttnArgs {
    const void* q;
    const void* k;
    const void* v;
    const void* arena;
    const long* kvmap;
    // Group descriptors (bf16 KVMap launches, optional): per frame, one
    // 2-word entry per 16-row copy group of the frame's key range, telling
    // which of the group's rows the map sends to the arena (format:
    // kvp_c_api.h, kvp_attn_forward_frames_gd). With them the kernel reads
    // map entries only for groups the entry cannot describe.
    const unsigned* gdesc;
    long gd_fstride;  // entries (word pairs) between frames' tables
    void* out;
    void* part_o;     // [splits][frames][nq][D] normalised partial O:
                      // fp16 from the bf16 kernel (row scaled by 2^e),
                      // fp32 from the fp32 kernel
    float* part_lse;  // [splits][frames][heads][nq] log2-sum-exp
    float* part_exp;  // [splits][frames][heads][nq] e of the fp16 row scale
    long q_fstride;   // elements between frames of q / out
    long kv_fstride;  // elements between frames of k / v
    long map_fstride; // entries between frames of kvmap
    long arena_fstride; // bytes between per-frame arena regions (0: one arena)
    // Key range of frame i of the launch: [max(key_begin, e - max_span), e)
    // with e = key_end + i * kend_step (kend_step = T for a causal layer
    // launch, 0 when every frame attends the same range).
    long key_begin;
    long key_end;
    long kend_step;
    long max_span;
    long keys_per_split;
    int nq;
    int D;
    int heads;
    int frames;
    int splits;
    int nqb;
    int layer_order;   // 1: XCD-column work order, frames longest first
    int xcd_slots;     // layer order: workgroups one XCD runs at once (0: unknown)
    int cyclic;        // layer order: the window cuts the ranges (walk order below)
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
    bool valid;
    bool rev;        // visit the key tiles last to first
    long start_key;  // >= 0: start the upward walk at the tile holding this key
};

// Number of (head, q-block) columns XCD x owns in the layer work order.
__host__ __device__ __forceinline__ int xcd_columns(int cols, int x) {
    return (x + 1) * cols / kNumXcd - x * cols / kNumXcd;
}

__device__ __forceinline__ WgCoord decode_wg(const AttnArgs& a) {
    WgCoord c;
    c.valid = true;
    c.split = 0;
    c.rev = false;
    c.start_key = -1;
    if (a.layer_order) {
        // Layer work order. The hardware hands workgroup b to XCD b % 8, so
        // XCD x runs workgroups x, x+8, x+16, ... in that order. XCD x owns
        // the contiguous (head, q-block) columns [x*C/8, (x+1)*C/8) and walks
        // them for every frame, last frame (longest key range) first: the
        // q-blocks and frames of one head, which all read that head's keys
        // from key 0 upward, share one L2, and the longest work starts first.
        const int cols = a.heads * a.nqb;
        const int x = (int)blockIdx.x % kNumXcd;
        const int j = (int)blockIdx.x / kNumXcd;
        const int n = xcd_columns(cols, x);
        if (n == 0 || j >= n * a.frames) {
            c.valid = false;
            c.qb = c.head = c.frame = 0;
            return c;
        }
        const int col = x * cols / kNumXcd + j % n;
        c.frame = a.frames - 1 - j / n;
        // Walk order, so that the workgroups an XCD runs together read the
        // same keys at the same time (one L2 fetch for all of them):
        // * ranges from a common first key (causal, no window): the first
        //   xcd_slots workgroups of an XCD start together and walk upward
        //   from that key in step. A later workgroup starts when an earlier
        //   one ends, with the long ranges still running near their top: it
        //   walks its keys downward from its range end, through the tiles
        //   the running workgroups fetched last (still in the L2), instead
        //   of restarting at the first key, whose tiles the L2 has evicted.
        // * ranges cut by a window (every frame's range starts one frame
        //   later than the next lower frame's): the workgroups of one round
        //   (xcd_slots consecutive ones, started and finished together since
        //   their ranges are equally long) all start at the first key of
        //   the round's highest frame (its first workgroup's), walk upward
        //   and wrap around to their own range start, so that they cross the
        //   keys the frames share in step.
        if (a.xcd_slots > 0) {
            if (!a.cyclic) {
                c.rev = j >= a.xcd_slots;
            } else {
                const int f_hi = a.frames - 1 - (j / a.xcd_slots) * a.xcd_slots / n;
                const long e = a.key_end + (long)f_hi * a.kend_step;
                const long b = e - a.max_span;
                c.start_key = b > a.key_begin ? b : a.key_begin;
            }
        }
        c.head = col / a.nqb;
        c.qb = col % a.nqb;
        return c;
    }
    int r = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    c.qb = r % a.nqb;
    r /= a.nqb;
    c.split = r % a.splits;
    r /= a.splits;
    c.head = r % a.heads;
    c.frame = r / a.heads;
    return c;
}

// Key range [kbeg, kend) of a workgroup: its frame's range, then its split.
__device__ __forceinline__ void wg_keys(const AttnArgs& a, const WgCoord& c, long& kbeg,
                                        long& kend) {
    const long e = a.key_end + (long)c.frame * a.kend_step;
    long b = e - a.max_span;
    if (b < a.key_begin) b = a.key_begin;
    kbeg = b + (long)c.split * a.keys_per_split;
    kend = kbeg + a.keys_per_split;
    if (kend > e) kend = e;
}

// Value of x held by lane (lane ^ 32).
__device__ __forceinline__ float other_half(float x) {
    return __shfl_xor(x, 32);
}

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

// fp32 kernel epilogue: writes the normalised result (or the fp32 split
// partial) of one wave. o[nb][v] holds O^T[d = 32*nb + 8*(v/4) + 4*hh + v%4][q].
__device__ __forceinline__ void store_rows_f32(const AttnArgs& a, const WgCoord& c, int q, int hh,
                                               const f32x16 (&o)[4], float m_run, float l_run) {
    if (q >= a.nq) return;
    const float inv_l = 1.0f / l_run;
    const int col0 = c.head * kHeadDim + 4 * hh;
    const bool split = a.splits > 1;
    const long slab = (long)c.split * a.frames + c.frame;
    float* dst = split ? static_cast<float*>(a.part_o) + (slab * a.nq + q) * (long)a.D + col0
                       : reinterpret_cast<float*>(a.out) + (long)c.frame * a.q_fstride +
                             (long)q * a.D + col0;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 w = {o[nb][4 * g + 0] * inv_l, o[nb][4 * g + 1] * inv_l,
                             o[nb][4 * g + 2] * inv_l, o[nb][4 * g + 3] * inv_l};
            *reinterpret_cast<f32x4*>(dst + 32 * nb + 8 * g) = w;
        }
    }
    if (split && hh == 0)
        a.part_lse[(slab * a.heads + c.head) * (long)a.nq + q] = m_run + __log2f(l_run);
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
//
// K and V tiles (64 keys x 128 dims, 16 KiB each) stream global -> LDS with
// buffer_load_dwordx4 ... lds (no register staging) into a two-stage ring:
// the loads of tile t+1 are in flight while tile t is computed. Lane l of the
// wave's load instruction writes LDS bytes [base + 16*l, +16); it picks the
// global 16-byte chunk that belongs at that (swizzled) LDS position.
//
// LDS layouts (row = key in tile, 256 B per row, 16 chunks of 16 B):
//   K: physical chunk = logical chunk ^ (row & 15)
//      (ds_read_b128 of 32 rows x one chunk is conflict free)
//   V: physical chunk = logical chunk ^ kVSwz[row & 3], kVSwz = {0,6,12,10}
//      (ds_read_b64_tr_b16 reads 4 consecutive rows x 32 B per 16-lane group;
//       the table keeps those 4 x 32 B on distinct banks for 32- and 64-bank
//       LDS models alike)
// ds_read_b64_tr_b16: in each 16-lane group, source lane 4s+r addresses row s,
// columns 4r..4r+3 of a 4 x 16 block; result lane j receives column j, rows
// 0..3. That yields the V^T operand of O^T = V^T P^T directly.
//
// Softmax: scores stay in the log2 domain (scale folded into one FMA before
// v_exp_f32). Exponentials are taken against the running max without
// computing the tile max; the running max is raised (and O, l rescaled
// together, wave-uniform branch) only when a tile's row sum would exceed the
// tile's key count (64) or is not finite — on the first tile and when scores
// rise above the running max. O/l is unchanged mathematically. Bounding
// each tile's sum by its key count bounds O by (keys so far) x max|V| and l
// by the key count, as the reference's update with every p <= 1 does
// (src/gated_attention_kernel.cu:101-115): fp32 O stays finite for every V
// the reference's stays finite for.
// ---------------------------------------------------------------------------

constexpr int kBf16TileBytes = kBf16BlockKeys * kHeadDim * 2;  // 16 KiB
// Raw buffer descriptor word 3 for gfx9-family (32-bit data format, no
// swizzle): out-of-range offsets (>= num_records) read as zero.
constexpr int kBufFlags = 0x00020000;
// Row-sum bound of one bf16 tile's exponentials: its key count (see the
// softmax note above).
constexpr float kRowSumLimit = (float)kBf16BlockKeys;
constexpr unsigned kVSwzTable = 0xAC60u;  // nibbles {0, 6, 12, 10}
// Buffer offset past the records of every bf16 tile descriptor (a tile
// covers at most 64 rows of 2*D bytes): a load there reads no memory and
// returns zeros.
constexpr unsigned kNoRecord = 0x80000000u;

typedef __attribute__((ext_vector_type(4))) short v4i16;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
#define KVP_LDS __attribute__((address_space(3)))

__device__ __forceinline__ unsigned vswz(int row) { return (kVSwzTable >> (4 * (row & 3))) & 15u; }

// s_waitcnt immediates (gfx9 encoding): vmcnt in [3:0] and [15:14],
// expcnt [6:4] = 7 and lgkmcnt [11:8] = 15 leave those counters alone.
constexpr int waitcnt_vm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

__device__ __forceinline__ void swap_halves(float x, float& lo, float& hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
}

// LDS access of the compute phase is written as inline asm on purpose: the
// K/V tiles arrive by asynchronous global->LDS copies (global_load_lds), and
// the compiler, unable to prove that a read of the current stage does not
// alias the copies in flight to the other stage, would otherwise wait for
// every outstanding copy (vmcnt(0)) before each read. Completion is tracked
// explicitly instead:
//   * vmcnt: before the barrier that publishes a stage, each wave waits for
//     its own copies of that stage (the next stage's copies stay in flight);
//   * lgkmcnt: each batch of LDS reads is waited for by an asm statement that
//     takes the destination registers as in/out operands, so no use of the
//     data can be scheduled before the wait.
// All these asm statements are volatile with a memory clobber, which keeps
// them in program order relative to one another and to the barrier.

__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int OFF>
__device__ __forceinline__ u32x4 lds_b128(unsigned addr) {
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF) : "memory");
    return r;
}

template <int OFF>
__device__ __forceinline__ unsigned lds_b32(unsigned addr) {
    unsigned r;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF) : "memory");
    return r;
}

template <int OFF>
__device__ __forceinline__ u32x2 lds_tr16(unsigned addr) {
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF) : "memory");
    return r;
}

__device__ __forceinline__ void lgkm_wait2(u32x4& a, u32x4& b) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b)::"memory");
}

// Waits for all but the two most recent LDS reads (LDS reads complete in
// issue order and no scalar-memory load is issued in the compute phase).
__device__ __forceinline__ void lgkm_wait2_keep2(u32x4& a, u32x4& b) {
    asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(a), "+v"(b)::"memory");
}

// fp32 kernel: wait for all but the newest LDS read / for all of them.
__device__ __forceinline__ void lgkm_wait_keep1(u32x4& a) {
    asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(a)::"memory");
}
__device__ __forceinline__ void lgkm_wait1x4(u32x4& a) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a)::"memory");
}
// fp32 kernel: wait for every LDS read, the 16 values of a V block among them.
__device__ __forceinline__ void lgkm_wait16(unsigned (&d)[16]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(d[4]), "+v"(d[5]),
                   "+v"(d[6]), "+v"(d[7]), "+v"(d[8]), "+v"(d[9]), "+v"(d[10]), "+v"(d[11]),
                   "+v"(d[12]), "+v"(d[13]), "+v"(d[14]), "+v"(d[15])::"memory");
}

// Waits until at most N LDS reads are outstanding.
template <int N>
__device__ __forceinline__ void lgkm_wait_tr_n(u32x2& a, u32x2& b, u32x2& c, u32x2& d) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N) : "memory");
}

// bf16 kernel epilogue: the wave's 32 query rows x 128 dims go out as
// 2-byte elements (fp16 split partials, or the bf16 output when the key range
// is not split). They are staged in LDS as query rows of 256 B (16-byte
// chunks XOR-swizzled by row & 15) and stored as full rows, 16 bytes per
// lane, instead of 8-byte pieces scattered over 32 rows. `stage` is 8 KiB of
// LDS that no other wave touches any more.
// An fp16 partial row is stored as P * 2^e with e chosen per query row so
// that its largest magnitude lies in [2^14, 2^15): every element keeps fp16's
// 11-bit precision relative to the row maximum whatever the scale of V (no
// overflow above 65504, no subnormal partials for tiny V); e goes to
// part_exp and the combine undoes it exactly.
template <typename T, bool kScaled>
__device__ __forceinline__ void store_rows_staged(const AttnArgs& a, const WgCoord& c, int wave,
                                                  int lane, const f32x16 (&o)[4], float m_run,
                                                  float l_run, unsigned char* stage) {
    typedef __attribute__((ext_vector_type(4))) T t4;
    const int lq = lane & 31;
    const int hh = lane >> 5;
    const int q0 = c.qb * kBlockQ + wave * 32;
    const float inv_l = 1.0f / l_run;
    int e = 0;
    if constexpr (kScaled) {
        float mx = 0.f;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int v = 0; v < 16; ++v) mx = fmaxf(mx, fabsf(o[nb][v]));
        mx = fmaxf(mx, other_half(mx)) * inv_l;
        if (mx > 0.f && mx <= 3.0e38f) e = 14 - ilogbf(mx);
    }
    auto cvt = [&](float x) -> T {
        const float y = x * inv_l;
        if constexpr (kScaled) return (T)__builtin_amdgcn_ldexpf(y, e);
        return (T)y;
    };
    unsigned char* wrow = stage + lq * 256;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const t4 w = {cvt(o[nb][4 * g + 0]), cvt(o[nb][4 * g + 1]), cvt(o[nb][4 * g + 2]),
                          cvt(o[nb][4 * g + 3])};
            const int pc = (4 * nb + g) ^ (lq & 15);
            *reinterpret_cast<t4*>(wrow + 16 * pc + 8 * hh) = w;
        }
    }
    const bool split = a.splits > 1;
    const long slab = (long)c.split * a.frames + c.frame;
    T* base = split ? static_cast<T*>(a.part_o) + slab * a.nq * (long)a.D
                    : reinterpret_cast<T*>(a.out) + (long)c.frame * a.q_fstride;
    base += c.head * kHeadDim;
    const int lc = lane & 15;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        const int row = 4 * it + (lane >> 4);
        const u32x4 v = *reinterpret_cast<const u32x4*>(stage + row * 256 + 16 * (lc ^ (row & 15)));
        const int q = q0 + row;
        if (q < a.nq) *reinterpret_cast<u32x4*>(base + (long)q * a.D + 8 * lc) = v;
    }
    const int q = q0 + lq;
    if (split && hh == 0 && q < a.nq) {
        const long i = (slab * a.heads + c.head) * (long)a.nq + q;
        a.part_lse[i] = m_run + __log2f(l_run);
        a.part_exp[i] = (float)e;
    }
}

// kMap: the launch reads a KVMap (a.kvmap != null); the map-free variant has
// no per-row source selection in its copy path.
// kColdNt (KVMap launches only): rows read from the original K/V buffers
// (not from the arena) are loaded non-temporally (the nt cache-policy bit),
// so the L2 evicts them first and keeps the arena's lines. An additive
// residency lever of this build: the reference's access-policy window
// (src/kv_tile_manager.cu:39-47) has hitRatio 1, so none of its accesses
// take the streaming miss property, and rows outside the window are cached
// normally there.
// kCyclic: the launch's ranges are cut by a window, and workgroups walk
// upward from their round's start key with a wrap (decode_wg); otherwise
// they walk upward from the range start, or downward when reversed.
// kGd (KVMap launches with group descriptors, a.gdesc): each wave reads its
// copy group's 8-byte descriptor per tile instead of the group's 16 map
// entries; only groups whose descriptor says "general" read the entries.
template <typename OutT, bool kMap, bool kColdNt, bool kCyclic, bool kGd = false>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_bf16_kernel(AttnArgs a) {
    static_assert(!kGd || (kMap && !kColdNt), "group descriptors serve the KVMap kernel");
    constexpr int kColdAux = kColdNt ? 2 : 0;  // buffer-load aux: bit 1 = nt
    __shared__ __attribute__((aligned(1024))) unsigned char k_lds0[kBf16TileBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char v_lds0[kBf16TileBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char k_lds1[kBf16TileBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char v_lds1[kBf16TileBytes];
    // Per-wave 2 KiB sink (KVMap kernel): the interleaved copies of a group
    // mixing arena and original rows land there (reading nothing), while
    // the group's own rows come from its per-lane copies.
    __shared__ __attribute__((aligned(1024))) unsigned char sink_lds[kMap ? 4 * 2048 : 16];

    const WgCoord c = decode_wg(a);
    if (!c.valid) return;  // whole workgroup: past the end of the layer order
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int hh = lane >> 5;
    // A wave whose 32 queries all lie past nq (the tail q-block of a frame)
    // only issues its share of the tile copies and joins the barriers.
    const bool active = c.qb * kBlockQ + wave * 32 < a.nq;

    long kbeg, kend;
    wg_keys(a, c, kbeg, kend);
    // keys of the range (key indices stay below 2^31: checked at launch)
    const int nkeys = (int)(kend - kbeg);
    const int ntiles = (nkeys + kBf16BlockKeys - 1) / kBf16BlockKeys;
    // Rows of tile t: 64 before the last tile, last_rows in it, none past
    // it (the loop prefetches past the end). Written as a choice between
    // loop-invariant values, so that it stays a scalar select (a clamp of
    // nkeys - 64*t becomes a vector min/max here, and a descriptor built
    // from a vector value is taken apart lane by lane).
    const int last_rows = nkeys - (ntiles - 1) * kBf16BlockKeys;
    // Tiles outside [0, ntiles) -- the loop's prefetches past either end of
    // the walk -- have no rows.
    auto tile_rows_x = [&](int t, int full, int last) {
        return (unsigned)t < (unsigned)(ntiles - 1) ? full : (t == ntiles - 1 ? last : 0);
    };
    // Key tile visited at loop step i (walk order: decode_wg): upward from
    // tile 0; downward from the last tile; or upward from the tile holding
    // start_key, wrapping to tile 0 after the last one. Steps past the walk
    // map outside [0, ntiles). The loop carries the map-entry and byte
    // offsets of the tiles it sets up as recurrences (one loop-invariant
    // step, less the range's tile span at the step where the walk wraps),
    // so that no 64-bit multiply enters the loop.
    int t_first = c.rev ? ntiles - 1 : 0;
    if (kCyclic && c.start_key >= kbeg && ntiles > 0) {
        const long st = (c.start_key - kbeg) / kBf16BlockKeys;
        t_first = st < ntiles ? (int)st : ntiles - 1;
    }
    const int t_dir = c.rev ? -1 : 1;
    const int wrap_at = ntiles - t_first;  // upward walks from t_first (kCyclic)
    auto tix = [&](int i) {
        const int t = t_first + t_dir * i;
        if constexpr (!kCyclic) return t;
        return i < wrap_at ? t : (i < ntiles ? t - ntiles : -1);
    };
    const long key_first = kbeg + (long)t_first * kBf16BlockKeys;
    const long key_step = (long)t_dir * kBf16BlockKeys;
    const long key_wrap = (long)ntiles * kBf16BlockKeys;
    // offset of step i+1's tile from step i's (i + 1 == wrap_at: the wrap)
    auto next_off = [&](long off, int i, long step, long wrap) {
        if constexpr (!kCyclic) return off + step;
        return off + step - (i + 1 == wrap_at ? wrap : 0L);
    };

    const __bf16* Q = reinterpret_cast<const __bf16*>(a.q) + (long)c.frame * a.q_fstride;
    const unsigned char* Kb = reinterpret_cast<const unsigned char*>(a.k) + 2L * c.frame * a.kv_fstride;
    const unsigned char* Vb = reinterpret_cast<const unsigned char*>(a.v) + 2L * c.frame * a.kv_fstride;
    const unsigned char* Ab =
        kMap ? reinterpret_cast<const unsigned char*>(a.arena) + (long)c.frame * a.arena_fstride
             : nullptr;
    const long* map = kMap ? a.kvmap + (long)c.frame * a.map_fstride : nullptr;
    const long row_bytes = 2L * a.D;
    const long hoff_b = 2L * c.head * kHeadDim;

    // Query fragment (B operand of S^T = K Q^T): Q[q][16*ks + 8*hh .. +8).
    const int q = c.qb * kBlockQ + wave * 32 + lq;
    const int qc = q < a.nq ? q : a.nq - 1;
    bf16x8 qf[8];
    {
        const __bf16* qp = Q + (long)qc * a.D + c.head * kHeadDim + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            qf[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qp + 16 * ks));
        // The Q loads stay in flight while the KVMap words and the first
        // tile's copies are issued; one wait below covers them all.
    }

    // Copy assignment: instruction i of wave w fills LDS bytes [(4w+i)*1 KiB, +1 KiB)
    // of each tile: rows 16w + 4i + lane/16, physical chunk lane % 16.
    // Copies are buffer loads straight into LDS. Per tile, the K/V buffer
    // descriptors are based at the tile's first key row and cover only rows
    // below kend, so rows past the end read as zeros (they are masked out of
    // the softmax) without any per-lane clamping; lane offsets are constant
    // across tiles. Arena rows (KVMap >= 0) go through an arena descriptor.
    const int ld_row0 = 16 * wave + (lane >> 4);
    const int ld_pch = lane & 15;
    const unsigned rb = (unsigned)row_bytes;
    // Rows ld_row0 + 4i: (row & 15) repeats with period 4 in i and (row & 3)
    // is the same for every i.
    unsigned kofs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        kofs[i] = (unsigned)hoff_b + 16u * ((unsigned)ld_pch ^ (unsigned)((ld_row0 + 4 * i) & 15));
    const unsigned vofs = (unsigned)hoff_b + 16u * ((unsigned)ld_pch ^ vswz(ld_row0));
    const unsigned lane_row = (unsigned)ld_row0 * rb;
    const __amdgpu_buffer_rsrc_t arena_rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(Ab), (short)0, -1, kBufFlags);

    // KVMap entries of a tile are loaded into registers two tiles ahead (one
    // 4-byte load per lane: lanes 0-31 of wave w hold the 32 words of the
    // tile's rows 16w..16w+15, entry e's low word in lane 2e and its high
    // word in lane 2e+1; words past the tile's end read as zeros). Right
    // before the tile's own K/V copies are issued they are decoded into
    // arena byte offsets; by then the load has landed (the loop waits for
    // all of a wave's loads at the top of each iteration). Arena rows are
    // addressed with 32-bit byte offsets from the arena base: an entry m is
    // used when its row ends within 4 GiB of that base
    // (2*(m+1)*row_bytes <= 2^32); any negative entry, or one beyond that,
    // reads the original K/V row (offset ~0u). Rows at or past the range end
    // take the original-row path too, whose descriptor reads them as zeros
    // (their map words are zero-filled padding, not entries).
    const unsigned max_arena_row = 0x80000000u / rb - 1u;
    // Wave-uniform: some row of the wave's 16-row copy group maps into the
    // arena. Almost every group holds none (an arena covers a few % of a
    // frame's keys), and then neither the per-row decode nor the per-lane
    // choice of source runs: the wave copies like the map-free kernel.
    bool grp_mapped = false;
    // Wave-uniform: every row of the group maps into the arena, to
    // consecutive arena rows (a run). Such a group copies like a plain
    // group, from the arena, without a per-lane choice of source (the frame
    // pipeline's layer arena holds mapped tiles in key order, so most fully
    // mapped groups are runs). Not in the non-temporal variant, whose hint
    // must reach original rows only.
    constexpr bool kRuns = kMap && !kColdNt;
    bool grp_run = false;
    unsigned run_base = 0;  // arena byte offset of a run's first row
    // arena byte offset of the lane's first copy row within a run
    const unsigned lane_arena = 2u * (unsigned)(lane >> 4) * rb;
    // hw: lane L < 32 holds word L of the wave's 16 entries (see above); an
    // entry can name an arena row only when its high word is 0.
    // A mapped group's copy i reads arena byte offset md[i] (lane's row
    // ld_row0 + 4i), or the original row where md[i] is ~0u; md is set only
    // for a mapped group (grp_mapped) and read only by its copies.
    auto decode_map = [&](int t, unsigned hw, unsigned (&md)[4]) {
        if constexpr (!kMap) return;
        // rows at or past the range end are zero-filled padding, not entries
        // (a tile outside the range has none)
        const int valid_rows = tile_rows_x(t, kBf16BlockKeys, last_rows);
        grp_mapped = __builtin_amdgcn_ballot_w64(lane < 32 && (lane & 1) && hw == 0u &&
                                                 16 * wave + (lane >> 1) < valid_rows) != 0;
        grp_run = false;
        if (__builtin_expect(!grp_mapped, 1)) return;
        if constexpr (kRuns) {
            // Lanes 0-31 already hold the group's 16 entries (entry e: low
            // word in lane 2e, high word in lane 2e+1). A run: all 16 rows
            // inside the range, every high word 0, low words l0 .. l0+15 with
            // the last row inside the reach of 32-bit offsets; then no
            // per-row decode.
            const unsigned l0 = (unsigned)__builtin_amdgcn_readlane((int)hw, 0);
            const bool full = 16 * wave + 16 <= valid_rows && l0 <= max_arena_row - 15u;
            const bool ok = lane >= 32 || ((lane & 1) ? hw == 0u : hw == l0 + (unsigned)(lane >> 1));
            if (full && __builtin_amdgcn_ballot_w64(!ok) == 0) {
                grp_run = true;
                run_base = 2u * l0 * rb;
#pragma unroll
                for (int i = 0; i < 4; ++i) md[i] = run_base + lane_arena + 8u * (unsigned)i * rb;
                return;
            }
        }
        // copy i of the lane takes row ld_row0 + 4i: entry (lane >> 4) + 4i,
        // words 2e and 2e+1 fetched from the lanes holding them (all eight
        // fetches in flight together, then one branch-free decode)
        unsigned lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = (lane >> 4) + 4 * i;
            lo[i] = (unsigned)__builtin_amdgcn_ds_bpermute(8 * e, (int)hw);
            hi[i] = (unsigned)__builtin_amdgcn_ds_bpermute(8 * e + 4, (int)hw);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool ok = (ld_row0 + 4 * i < valid_rows) & (hi[i] == 0u) &
                            (lo[i] <= max_arena_row);
            md[i] = ok ? 2u * lo[i] * rb : ~0u;
        }
    };
    // the map words of tile t, whose first key is t0 (see above); zeros
    // outside the range
    auto load_map_tile = [&](int t, long t0) -> unsigned {
        if constexpr (!kMap) return ~0u;
        // outside the range (at most two tiles beyond either end) the base
        // is past the slice, but the descriptor has no records to read
        const int nrec = tile_rows_x(t, kBf16BlockKeys * 8, last_rows * 8);
        const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<long*>(map + t0), (short)0, nrec, kBufFlags);
        return __builtin_amdgcn_raw_buffer_load_b32(mrs, 128u * wave + 4u * lane, 0, 0);
    };
    // the map words of step i's tile
    auto load_map = [&](int i, long t0) -> unsigned { return load_map_tile(tix(i), t0); };

    // Group descriptors (kGd): entry 4*t + w of the workgroup's table
    // describes rows 16w..16w+15 of tile t, i.e. wave w's copy group. The
    // table starts at the workgroup's first key (a split starts a multiple
    // of 64 keys into its frame's range) and its descriptor covers exactly
    // the tiles of the range, so the loop's prefetches past either end of
    // the walk read zeros ("no arena row").
    const unsigned* gdf =
        kGd ? a.gdesc + 2L * c.frame * a.gd_fstride + 2L * ((long)c.split * a.keys_per_split / 16)
            : nullptr;
    const __amdgpu_buffer_rsrc_t gd_rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned*>(gdf), (short)0, kGd ? ntiles * 32 : 0, kBufFlags);
    // step i's descriptor: even lanes load its word 0, odd lanes word 1
    // (prep_gd takes them from lanes 0 and 1). Per-lane offsets on
    // purpose: a load whose address the compiler sees as uniform counts as a
    // uniform value, and the copy descriptors derived from it then end up in
    // VGPRs, each copy wrapped in a lane-by-lane (waterfall) loop.
    auto load_gd = [&](int i) -> unsigned {
        if constexpr (!kGd) return 0u;
        // a tile index below 0 wraps the offset far past the records
        const unsigned off = (unsigned)(4 * tix(i) + wave) * 8u + 4u * (unsigned)(lane & 1);
        return __builtin_amdgcn_raw_buffer_load_b32(gd_rs, off, 0, 0);
    };
    // Row rr (0..15) of the group against a sub-run word w (bit 31 set:
    // rows r0..r0+n-1 map to arena rows l..l+n-1): the arena byte offset of
    // the row's arena row, or `off` unchanged when the row is not in the
    // sub-run, lies past the range end, or its arena row is beyond the reach
    // of 32-bit offsets (such rows read the original row, as in decode_map).
    auto sub_run = [&](unsigned w, unsigned rr, unsigned row_ok, unsigned off) -> unsigned {
        const unsigned l = w & 0x7FFFFFu;
        const unsigned r0 = (w >> 23) & 15u;
        const unsigned n = ((w >> 27) & 15u) + 1u;
        const unsigned m = l + (rr - r0);
        const bool in = (w >> 31) != 0u && rr - r0 < n && m <= max_arena_row && row_ok != 0u;
        return in ? 2u * m * rb : off;
    };
    // A tile's copies are set up by prep_tile (descriptors and LDS bases)
    // and issued as 4 K/V pairs. Issued back to back, a wave's 8 copies
    // (1 KiB each) kept it stalled on instruction issue for about a quarter
    // of every tile on MI355X, while both workgroups of the CU pushed their
    // 64 KiB through the load path at once; the main loop instead issues one
    // pair after every second QK k-step of the tile being computed, so the
    // copies trickle out between MFMAs (copy_plain).
    // copy_plain(i) reads K at cp_k + i*cp_step + kofs[i] and V at
    // cp_v + i*cp_step + vofs through krs / vrs into LDS bytes pk + i*pstep
    // and pv + i*pstep. For a plain group (no KVMap entry) krs / vrs cover
    // the tile's K / V rows; for a run they both start at the run's first
    // arena row; for a mixed group (copy_pair fills its rows) the offsets lie
    // past the tile's records, so these copies read nothing, and they land
    // in the wave's sink.
    __amdgpu_buffer_rsrc_t krs, vrs;
    unsigned koff = 0, voff = 0;
    unsigned cp_k = lane_row, cp_v = lane_row, cp_step = 4u * rb;
    unsigned pk = 0, pv = 0, pstep = 1024u;
    const unsigned sink = (unsigned)(uintptr_t)sink_lds + 2048u * (unsigned)wave;
    const unsigned lane_arena_v = lane_arena + rb;
    // step i's tile starts kvo bytes into the frame's K / V
    auto prep_tile = [&](int i, long kvo, unsigned char* kdst, unsigned char* vdst) {
        const int t = tix(i);
        const unsigned char* kb = Kb + kvo;
        const unsigned char* vb = Vb + kvo;
        // tiles outside the range (the loop's trailing copies) cover no rows
        const int nrec = tile_rows_x(t, kBf16BlockKeys * (int)rb, last_rows * (int)rb);
        krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(kb), (short)0, nrec,
                                                kBufFlags);
        vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(vb), (short)0, nrec,
                                                kBufFlags);
        koff = (unsigned)__builtin_amdgcn_readfirstlane((int)(uintptr_t)kdst) + 4096u * wave;
        voff = (unsigned)__builtin_amdgcn_readfirstlane((int)(uintptr_t)vdst) + 4096u * wave;
        cp_k = lane_row;
        cp_v = lane_row;
        cp_step = 4u * rb;
        pk = koff;
        pv = voff;
        pstep = 1024u;
        if (kRuns && grp_run) {
            // a run's [K row | V row] arena rows: 2*rb apart, V rb after K
            krs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<unsigned char*>(Ab + run_base), (short)0, -1, kBufFlags);
            vrs = krs;
            cp_k = lane_arena;
            cp_v = lane_arena_v;
            cp_step = 8u * rb;
        } else if (kMap && grp_mapped) {
            cp_k = kNoRecord;
            cp_v = kNoRecord;
            cp_step = 0;
            pk = sink;
            pv = sink + 1024u;
            pstep = 0;
        }
    };
    auto copy_plain = [&](int i) {
        KVP_LDS void* kd = (KVP_LDS void*)(uintptr_t)(pk + pstep * (unsigned)i);
        KVP_LDS void* vd = (KVP_LDS void*)(uintptr_t)(pv + pstep * (unsigned)i);
        const unsigned step = (unsigned)i * cp_step;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, kd, 16, cp_k + step + kofs[i], 0, 0,
                                                 kColdAux);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, vd, 16, cp_v + step + vofs, 0, 0, kColdAux);
    };
    // Copy pair i of any group: each row's source chosen per lane (arena
    // row where decode_map set an offset, else the original row).
    auto copy_pair = [&](int i, const unsigned (&md)[4]) {
        KVP_LDS void* kd = (KVP_LDS void*)(uintptr_t)(koff + 1024u * i);
        KVP_LDS void* vd = (KVP_LDS void*)(uintptr_t)(voff + 1024u * i);
        const unsigned row_off = lane_row + 4u * i * rb;
        if (kMap && md[i] != ~0u) {
            const unsigned ao = md[i];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(arena_rs, kd, 16, ao + kofs[i], 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(arena_rs, vd, 16, ao + rb + vofs, 0, 0, 0);
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, kd, 16, row_off + kofs[i], 0, 0,
                                                     kColdAux);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, vd, 16, row_off + vofs, 0, 0,
                                                     kColdAux);
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[nb][v] = 0.f;
    float m_run = -INFINITY;
    float l_run = 0.f;
    const float cl2 = a.scale_log2;

    // Row sums of a tile's P on the matrix core: P^T fragment g (the B
    // operand of the PV MFMA: lane l holds keys 16g + 8*(l/32) + 0..7 of
    // query l % 32) read as the B operand of a 16x16x32 MFMA puts those
    // values in row group k/8 = l/16 of column n = l % 16. With A[m][k] = 1
    // where bit 0 of k/8 equals bit 0 of m (else 0), D[m][n] sums the 16 keys
    // of query n (m even: lanes n and n+32) or of query n + 16 (m odd: lanes
    // n+16 and n+48); lane l reads D[4*(l/16) + v][l % 16] in acc[v], so its
    // own query's sum is acc[(l/16) & 1]. Four such MFMAs (one per k-step)
    // replace 32 VALU adds and a cross-half exchange per tile, and the sum
    // is of the bf16 weights the PV product uses.
    const bool rs_hi = (lane >> 4) & 1;
    bf16x8 rsel;
#pragma unroll
    for (int i = 0; i < 8; ++i) rsel[i] = (((lane >> 4) ^ lane) & 1) ? (__bf16)0.f : (__bf16)1.f;

    // Per-lane parts of the LDS read addresses.
    const unsigned kswz = (unsigned)(lq & 15);
    const int grp = lane >> 4;
    const int tr_s = (lane & 15) >> 2;
    const int tr_r = lane & 3;
    const unsigned vs = vswz(tr_s);
    const int vsub = 8 * (tr_r & 1);
    const unsigned vcl = (unsigned)(2 * (grp & 1) + (tr_r >> 1));  // chunk bits below 4*nb

    // `between(ks)` runs after the MFMAs of QK k-step ks (the next tile's
    // copies are issued there).
    auto compute_tile = [&](int t, const unsigned char* ks_lds, const unsigned char* vt_lds,
                            auto&& between) {
        const unsigned kbase = (unsigned)(uintptr_t)ks_lds + (unsigned)(lq * 256);
        f32x16 s0, s1;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            s0[v] = 0.f;
            s1[v] = 0.f;
        }
        // S^T = K Q^T; K fragments are read two k-steps ahead of their MFMAs
        // (lgkmcnt(2) leaves the newest pair in flight).
        u32x4 ka[3], kb[3];
        // MFMA sections run at raised wave priority: when both waves of a
        // SIMD are ready, the one feeding the matrix core issues first and
        // the other's softmax VALU work fills the gaps.
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const unsigned ad = kbase + ((((unsigned)(2 * ks + hh)) ^ kswz) << 4);
            ka[ks] = lds_b128<0>(ad);
            kb[ks] = lds_b128<32 * 256>(ad);
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int cur = ks % 3;
            if (ks + 1 < 8)
                lgkm_wait2_keep2(ka[cur], kb[cur]);
            else
                lgkm_wait2(ka[cur], kb[cur]);
            if (ks + 2 < 8) {
                const int nx = (ks + 2) % 3;
                const unsigned ad = kbase + ((((unsigned)(2 * (ks + 2) + hh)) ^ kswz) << 4);
                ka[nx] = lds_b128<0>(ad);
                kb[nx] = lds_b128<32 * 256>(ad);
            }
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ka[cur]),
                                                         qf[ks], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kb[cur]),
                                                         qf[ks], s1, 0, 0, 0);
            between(ks);
        }

        __builtin_amdgcn_s_setprio(0);

        // O^T += V^T P^T reads V^T fragments with transposing LDS reads of
        // rows 16g + 4hh + s and +8 (row offsets 16g*256 and 8*256 are
        // immediates): 8 reads per 32-column block nb, in two groups of 4
        // that feed 2 MFMAs each. Block 0 is read now, ahead of the softmax;
        // each later group is read one block ahead of its MFMAs.
        const unsigned vbase = (unsigned)(uintptr_t)vt_lds + (unsigned)((4 * hh + tr_s) * 256 + vsub);
        auto vaddr = [&](int nb) { return vbase + ((((unsigned)(4 * nb) | vcl) ^ vs) << 4); };
        u32x2 vr[2][8];
        auto read_v = [&](u32x2* d, int nb, int half) {
            const unsigned ad = vaddr(nb);
            if (half == 0) {
                d[0] = lds_tr16<0>(ad);
                d[1] = lds_tr16<8 * 256>(ad);
                d[2] = lds_tr16<16 * 256>(ad);
                d[3] = lds_tr16<24 * 256>(ad);
            } else {
                d[4] = lds_tr16<32 * 256>(ad);
                d[5] = lds_tr16<40 * 256>(ad);
                d[6] = lds_tr16<48 * 256>(ad);
                d[7] = lds_tr16<56 * 256>(ad);
            }
        };
        read_v(vr[0], 0, 0);
        read_v(vr[0], 0, 1);

        float s[32];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            s[v] = s0[v];
            s[16 + v] = s1[v];
        }
        const int left = nkeys - t * kBf16BlockKeys;
        if (left < kBf16BlockKeys) {
            // s[v] holds key kc(v) + 4*hh of the tile, kc(v) a compile-time
            // constant: comparing kc(v) with lim - 4*hh keeps the per-lane
            // key indices out of registers.
            const int lim = left - 4 * hh;
#pragma unroll
            for (int v = 0; v < 32; ++v) {
                const int kc = 32 * (v >> 4) + 8 * ((v & 15) >> 2) + (v & 3);
                if (kc >= lim) s[v] = -INFINITY;
            }
        }

        // Exponentiate against the running max; only when the tile's row sum
        // overflows the bound (first tile, where the running max is -inf, or
        // scores that grew far beyond it) take the slow path: raise the max
        // to the tile max, rescale O and l, and exponentiate again.
        // The tile's row sum comes from the matrix core (rsel above), so
        // the VALU work per score is one FMA, one exponential and half a
        // bf16 pack. (A 0 x inf product in that sum, from an infinite
        // exponential, yields NaN, which fails the bound check as the inf
        // itself would.)
        bf16x8 pb[4];
        auto exp_tile = [&](float mref) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    const float e0 = fast_exp2(fmaf(s[8 * g + i], cl2, -mref));
                    const float e1 = fast_exp2(fmaf(s[8 * g + i + 1], cl2, -mref));
                    pb[g][i] = (__bf16)e0;
                    pb[g][i + 1] = (__bf16)e1;
                }
            }
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int g = 0; g < 4; ++g)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rsel, pb[g], acc, 0, 0, 0);
            return rs_hi ? acc[1] : acc[0];
        };
        float tot = exp_tile(m_run);
        if (__builtin_amdgcn_ballot_w64(!(tot <= kRowSumLimit))) {
            float mx = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
            for (int v = 3; v < 31; v += 2) mx = fmaxf(fmaxf(mx, s[v]), s[v + 1]);
            mx = fmaxf(mx, s[31]);
            float mlo, mhi;
            swap_halves(mx, mlo, mhi);
            const float m_new = fmaxf(m_run, fmaxf(mlo, mhi) * cl2);
            const float corr = fast_exp2(m_run - m_new);  // 0 while m_run is -inf
            l_run *= corr;
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[nb][v] *= corr;
            m_run = m_new;
            tot = exp_tile(m_run);
        }
        l_run += tot;

        // LDS reads complete in issue order, so lgkmcnt(4) waits for the
        // older of the two groups in flight.
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            u32x2* cur = vr[nb & 1];
            u32x2* nxt = vr[(nb + 1) & 1];
            lgkm_wait_tr_n<4>(cur[0], cur[1], cur[2], cur[3]);
            if (nb < 3) read_v(nxt, nb + 1, 0);
            const u32x4 va0 = {cur[0][0], cur[0][1], cur[1][0], cur[1][1]};
            const u32x4 va1 = {cur[2][0], cur[2][1], cur[3][0], cur[3][1]};
            o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, va0), pb[0],
                                                            o[nb], 0, 0, 0);
            o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, va1), pb[1],
                                                            o[nb], 0, 0, 0);
            if (nb < 3) {
                lgkm_wait_tr_n<4>(cur[4], cur[5], cur[6], cur[7]);
                read_v(nxt, nb + 1, 1);
            } else {
                lgkm_wait_tr_n<0>(cur[4], cur[5], cur[6], cur[7]);
            }
            const u32x4 va2 = {cur[4][0], cur[4][1], cur[5][0], cur[5][1]};
            const u32x4 va3 = {cur[6][0], cur[6][1], cur[7][0], cur[7][1]};
            o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, va2), pb[2],
                                                            o[nb], 0, 0, 0);
            o[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, va3), pb[3],
                                                            o[nb], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    };

    unsigned hw_next = ~0u;  // map words of the tile after the next one
    // first key of the next map load's tile, byte offset of the next
    // prep_tile's tile
    long map_next = next_off(key_first, 0, key_step, key_wrap);
    const long kv_step = key_step * (long)rb;
    const long kv_wrap = key_wrap * (long)rb;
    long kv_next = key_first * (long)rb;

    // ---- copies of a descriptor launch (kGd) ----
    // Copy i of a wave moves rows 4i..4i+3 of its 16-row group (row
    // 4i + (lane >> 4), chunk lane & 15, as in copy_plain) with
    // raw buffer loads whose lane offset is row x pitch + chunk: an original
    // row (pitch rb, descriptor based at the group's first row) or an arena
    // row ([K row | V row], pitch 2 rb, descriptor based at arena row l - r0
    // of the sub-run), the pitch and the descriptor chosen per copy by
    // scalar selects. Rows at or past the range end lie past the original
    // descriptor's records and read as zeros. (Structured-buffer loads, index
    // x stride in the descriptor, need no per-copy lane arithmetic, but with
    // them the windowed launch read 25 % more fabric bytes per frame than
    // with these.)
    // byte offset of copy i's row at the original pitch: row 4i +
    // (lane >> 4) of the group, times rb; the arena pitch (2 rb) is this
    // shifted left by one, so a copy's lane offset is one shift-and-add of a
    // loop-invariant value (a per-copy row x pitch multiply is a quarter-rate
    // VALU op)
    unsigned grow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) grow[i] = (unsigned)(4 * i + (lane >> 4)) * rb;
    // the step being set up (prep_gd): its original rows, the arena sub-run
    // its copies may take, which of the 4 copies take it, and what the slow
    // path needs
    const unsigned char* go_k = Kb;
    const unsigned char* go_v = Vb;
    int go_n = 0;                     // rows of the group inside the range
    const unsigned char* ga_k = Ab;   // K part of arena row (l - r0) of the sub-run
    unsigned gsel = 0;                // bit i: copy i reads the sub-run
    bool gslow = false;               // some rows need a per-row source
    unsigned gw0 = 0, gw1 = 0;        // the descriptor words (slow path)
    int gt = 0;                       // the step's tile
    long gkey0 = 0;                   // its first key (slow path: map words)
    unsigned gkoff = 0, gvoff = 0;    // LDS bases of the wave's copies
    // Step i's group of tile t (first key key0, K/V byte offset kvo) from its
    // descriptor g (decoded from lanes 0 and 1), copies into kdst / vdst. The
    // fast form: no arena row, or one sub-run whose rows start and end on
    // 4-row copy boundaries (every policy tile of the frame pipeline's layer
    // arena, whose frames start on 4-row boundaries); anything else copies
    // the original rows and fixes the mapped ones up afterwards (overwrite_gd).
    // Every value is a select, not assigned under a branch: branch-assigned,
    // the compiler takes such values for divergent, moves the descriptors
    // built from them into VGPRs and wraps every copy in a lane-by-lane loop.
    auto prep_gd = [&](int t, long kvo, long key0, unsigned char* kdst, unsigned char* vdst,
                       unsigned g) {
        const unsigned w0 = (unsigned)__builtin_amdgcn_readlane((int)g, 0);
        const unsigned w1 = (unsigned)__builtin_amdgcn_readlane((int)g, 1);
        const int rows = tile_rows_x(t, kBf16BlockKeys, last_rows) - 16 * wave;
        const int grows = rows < 0 ? 0 : (rows > 16 ? 16 : rows);
        const long goff = kvo + 16L * wave * (long)rb;
        go_k = Kb + goff;
        go_v = Vb + goff;
        go_n = grows;
        const unsigned l = w0 & 0x7FFFFFu;
        const unsigned r0 = (w0 >> 23) & 15u;
        const unsigned n = ((w0 >> 27) & 15u) + 1u;
        const bool fast = (w0 >> 31) != 0u && w1 == 0u && ((r0 | n) & 3u) == 0u &&
                          (int)(r0 + n) <= grows && l + n - 1u <= max_arena_row;
        gsel = fast ? ((1u << (n >> 2)) - 1u) << (r0 >> 2) : 0u;
        ga_k = Ab + 2L * (long)rb * ((long)l - (long)r0);
        gslow = w0 != 0u && !fast;
        gw0 = w0;
        gw1 = w1;
        gt = t;
        gkey0 = key0;
        gkoff = (unsigned)__builtin_amdgcn_readfirstlane((int)(uintptr_t)kdst) + 4096u * wave;
        gvoff = (unsigned)__builtin_amdgcn_readfirstlane((int)(uintptr_t)vdst) + 4096u * wave;
    };
    auto copy_gd = [&](int i) {
        // descriptors built per copy from a few scalars (four of them held
        // across the tile's MFMAs pushed SGPR spills into the loop)
        const bool ar = ((gsel >> i) & 1u) != 0u;
        const int nrec = ar ? 0x7fffffff : go_n * (int)rb;
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<unsigned char*>(ar ? ga_k : go_k), (short)0, nrec, kBufFlags);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<unsigned char*>(ar ? ga_k + rb : go_v), (short)0, nrec, kBufFlags);
        // (a select between precomputed offsets of both pitches put those
        // arrays in scratch memory)
        const unsigned row = grow[i] << (ar ? 1u : 0u);
        KVP_LDS void* kd = (KVP_LDS void*)(uintptr_t)(gkoff + 1024u * (unsigned)i);
        KVP_LDS void* vd = (KVP_LDS void*)(uintptr_t)(gvoff + 1024u * (unsigned)i);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, kd, 16, row + kofs[i], 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, vd, 16, row + vofs, 0, 0, 0);
    };
    // The slow path of the step prep_gd set up last, after its 4 copies were
    // issued: each row the map sends to the arena is copied again from its
    // arena row into the same LDS row. A wave's loads complete in issue
    // order, so the arena row lands last. Sources: the sub-run words, or for
    // a general group the tile's map words (loaded now).
    auto overwrite_gd = [&]() {
        if (__builtin_expect(!gslow, 1)) return;
        unsigned md[4] = {~0u, ~0u, ~0u, ~0u};
        if (gw0 == 1u) {
            decode_map(gt, load_map_tile(gt, gkey0), md);
        } else {
            const int valid_rows = tile_rows_x(gt, kBf16BlockKeys, last_rows);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned rr = (unsigned)((lane >> 4) + 4 * i);
                const unsigned ok = ld_row0 + 4 * i < valid_rows ? 1u : 0u;
                md[i] = sub_run(gw1, rr, ok, sub_run(gw0, rr, ok, ~0u));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (md[i] != ~0u) {
                KVP_LDS void* kd = (KVP_LDS void*)(uintptr_t)(gkoff + 1024u * (unsigned)i);
                KVP_LDS void* vd = (KVP_LDS void*)(uintptr_t)(gvoff + 1024u * (unsigned)i);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(arena_rs, kd, 16, md[i] + kofs[i], 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(arena_rs, vd, 16, md[i] + rb + vofs, 0, 0,
                                                         0);
            }
        }
    };

    if constexpr (kGd) {
        // Step t+2 is set up at the end of step t (after its MFMAs, where the
        // wave would otherwise wait at the next barrier): its descriptor,
        // loaded one step earlier, its copy parameters (into the stage step t
        // read; the copies are issued after the barrier) and the load of step
        // t+3's descriptor.
        unsigned gd_next = 0u;
        long gd_key = key_first;
        if (ntiles > 0) {
            const unsigned g0 = load_gd(0);
            const unsigned g1 = load_gd(1);
            prep_gd(tix(0), kv_next, gd_key, k_lds0, v_lds0, g0);
            kv_next = next_off(kv_next, 0, kv_step, kv_wrap);
            gd_key = next_off(gd_key, 0, key_step, key_wrap);
#pragma unroll
            for (int i = 0; i < 4; ++i) copy_gd(i);
            overwrite_gd();
            prep_gd(tix(1), kv_next, gd_key, k_lds1, v_lds1, g1);
            kv_next = next_off(kv_next, 1, kv_step, kv_wrap);
            gd_key = next_off(gd_key, 1, key_step, key_wrap);
            gd_next = load_gd(2);
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        for (int t = 0; t < ntiles; ++t) {
            unsigned char* kcur = (t & 1) ? k_lds1 : k_lds0;
            unsigned char* vcur = (t & 1) ? v_lds1 : v_lds0;
            // The newest vector-memory operation of the wave is the
            // descriptor load issued at the end of the previous step (used
            // one step later); everything before it -- this tile's copies and
            // overwrites -- has landed once at most one is outstanding (a
            // wave's vector-memory operations complete in issue order).
            // Waiting for all of them would expose that load's latency on
            // every tile.
            wait_vm<1>();
            wg_barrier();
            if (active) {
                compute_tile(tix(t), kcur, vcur, [&](int ks) {
                    if ((ks & 1) == 0) copy_gd(ks >> 1);
                });
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) copy_gd(i);
            }
            overwrite_gd();
            prep_gd(tix(t + 2), kv_next, gd_key, kcur, vcur, gd_next);
            kv_next = next_off(kv_next, t + 2, kv_step, kv_wrap);
            gd_key = next_off(gd_key, t + 2, key_step, key_wrap);
            gd_next = load_gd(t + 3);
        }
    } else {
        if (ntiles > 0) {
            const unsigned hw0 = load_map(0, key_first);
            hw_next = load_map(1, map_next);
            map_next = next_off(map_next, 1, key_step, key_wrap);
            unsigned md[4] = {~0u, ~0u, ~0u, ~0u};
            decode_map(tix(0), hw0, md);
            prep_tile(0, kv_next, k_lds0, v_lds0);
            kv_next = next_off(kv_next, 0, kv_step, kv_wrap);
#pragma unroll
            for (int i = 0; i < 4; ++i) copy_pair(i, md);
        }
        // Compiler-visible wait for every load so far (Q, map, tile 0): the
        // loop then never waits for vector memory on the Q registers' account.
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        for (int t = 0; t < ntiles; ++t) {
            // t counts loop steps; step t computes tile tix(t). Step t's tile
            // lives in stage t & 1; step t+1's tile streams into the other
            // stage, which held step t-1's: every wave finished reading it
            // before it reached the barrier below, so one barrier per tile
            // suffices
            unsigned char* kcur = (t & 1) ? k_lds1 : k_lds0;
            unsigned char* vcur = (t & 1) ? v_lds1 : v_lds0;
            unsigned char* knext = (t & 1) ? k_lds0 : k_lds1;
            unsigned char* vnext = (t & 1) ? v_lds0 : v_lds1;
            // each wave's copies of step t's tile (and its map load) have
            // landed, then the barrier publishes the whole tile
            wait_vm<0>();
            wg_barrier();
            // The copies for step t+1 and the map load for step t+2 are issued
            // unconditionally, so the QK k-steps they sit between stay one
            // basic block: past the end of the walk the descriptors cover no
            // rows (every row and map word reads as zero) and no KVMap entry
            // is decoded (rows outside the range are not entries).
            const unsigned hw1 = hw_next;
            hw_next = load_map(t + 2, map_next);
            map_next = next_off(map_next, t + 2, key_step, key_wrap);
            unsigned md[4];
            decode_map(tix(t + 1), hw1, md);
            prep_tile(t + 1, kv_next, knext, vnext);
            kv_next = next_off(kv_next, t + 1, kv_step, kv_wrap);
            // wave-uniform: the group mixes arena and original rows, each
            // row's source chosen per lane (copy_pair)
            const bool mixed = kMap && grp_mapped && !(kRuns && grp_run);
            if (active) {
                if (__builtin_expect(mixed, 0)) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) copy_pair(i, md);
                }
                compute_tile(tix(t), kcur, vcur, [&](int ks) {
                    if ((ks & 1) == 0) copy_plain(ks >> 1);
                });
            } else if (mixed) {
#pragma unroll
                for (int i = 0; i < 4; ++i) copy_pair(i, md);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) copy_plain(i);
            }
        }
    }
    // the trailing copies land before the workgroup's LDS is released, and
    // every wave has read its last tile before the epilogue stages output
    // rows there
    wait_vm<0>();
    wg_barrier();
    if (!active) return;

    // Stage in the last tile's stage: every wave has passed the barrier
    // after its last read, and the trailing copies target the other stage.
    unsigned char* last_k = (ntiles > 0 && ((ntiles - 1) & 1)) ? k_lds1 : k_lds0;
    unsigned char* last_v = (ntiles > 0 && ((ntiles - 1) & 1)) ? v_lds1 : v_lds0;
    unsigned char* stage = (wave < 2 ? last_k : last_v) + 8192 * (wave & 1);
    if (a.splits > 1)
        store_rows_staged<_Float16, true>(a, c, wave, lane, o, m_run, l_run, stage);
    else
        store_rows_staged<OutT, false>(a, c, wave, lane, o, m_run, l_run, stage);
}

// ---------------------------------------------------------------------------
// fp32 kernel
//
// Same decomposition as the bf16 kernel (4 waves x 32 queries per
// workgroup), v_mfma_f32_32x32x2_f32, 32-key tiles. K and V tiles (32 keys x
// 128 dims, 16 KiB each) stream global -> LDS with buffer_load_dwordx4 ...
// lds into a two-stage ring; the copies of tile t+1 go out between the QK
// MFMAs of tile t. An LDS row is one key's 512 bytes (32 chunks of 16 B):
//   K: physical chunk = logical ^ (row & 15): the ds_read_b128 of 32 rows x
//      one chunk is conflict free;
//   V: physical chunk = logical ^ 8*((row >> 2) & 1): the ds_read_b32 of
//      rows r and r+4 x 32 columns lands on all 64 banks once.
// Copy i (0..3) of wave w fills bytes [(4w+i) KiB, +1 KiB) of a K (and a V)
// stage: rows 8w + 2i + lane/32, physical chunk lane % 32. Rows past the
// range end read zeros through the tile's buffer descriptor. With a KVMap,
// a row whose entry m >= 0 is copied from arena row m instead, through a
// 64-bit address per lane; the entries of tile t+2 are loaded into
// registers during tile t.
// Softmax as in the bf16 kernel: exponentials against the running max, the
// max raised (and O, l rescaled) only when a tile's row sum exceeds the
// tile's key count (32) or is not finite; P stays fp32.
// ---------------------------------------------------------------------------

// Row-sum bound of one fp32 tile's exponentials: its key count.
constexpr float kF32RowSumLimit = (float)kF32BlockKeys;
constexpr int kF32TileBytes = kF32BlockKeys * kHeadDim * 4;  // 16 KiB

template <bool kMap>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_f32_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(1024))) unsigned char k_lds0[kF32TileBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char v_lds0[kF32TileBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char k_lds1[kF32TileBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char v_lds1[kF32TileBytes];

    const WgCoord c = decode_wg(a);
    if (!c.valid) return;  // whole workgroup: past the end of the layer order
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lq = lane & 31;
    const int hh = lane >> 5;
    // waves with no valid query issue their share of each tile's copies and
    // skip the MFMAs
    const bool active = c.qb * kBlockQ + wave * 32 < a.nq;

    long kbeg, kend;
    wg_keys(a, c, kbeg, kend);
    const int ntiles = (int)((kend - kbeg + kF32BlockKeys - 1) / kF32BlockKeys);

    const float* Q = reinterpret_cast<const float*>(a.q) + (long)c.frame * a.q_fstride;
    const unsigned char* Kb = reinterpret_cast<const unsigned char*>(a.k) + 4L * c.frame * a.kv_fstride;
    const unsigned char* Vb = reinterpret_cast<const unsigned char*>(a.v) + 4L * c.frame * a.kv_fstride;
    const unsigned char* Ab =
        kMap ? reinterpret_cast<const unsigned char*>(a.arena) + (long)c.frame * a.arena_fstride
             : nullptr;
    const long* map = kMap ? a.kvmap + (long)c.frame * a.map_fstride : nullptr;
    const long D = a.D;
    const long row_bytes = 4L * D;
    const unsigned rb = (unsigned)row_bytes;
    const long hoff_b = 4L * c.head * kHeadDim;

    // Query fragment: lane holds Q[q][8*j + 4*hh .. +4) for j = 0..15;
    // MFMA k-step (j, i) pairs head dim 8*j + 4*hh + i of both operands.
    const int q = c.qb * kBlockQ + wave * 32 + lq;
    const int qc = q < a.nq ? q : a.nq - 1;
    f32x4 qf[16];
    {
        const float* qp = Q + (long)qc * D + c.head * kHeadDim + 4 * hh;
#pragma unroll
        for (int j = 0; j < 16; ++j) qf[j] = *reinterpret_cast<const f32x4*>(qp + 8 * j);
    }

    // Copy geometry: copy i of this lane moves tile row 8w + 2i + lane/32,
    // physical chunk lane % 32.
    const int pch = lane & 31;
    auto cp_row = [&](int i) { return 8 * wave + 2 * i + (lane >> 5); };
    auto k_chunk = [&](int i) { return pch ^ (cp_row(i) & 15); };
    auto v_chunk = [&](int i) { return pch ^ (((cp_row(i) >> 2) & 1) << 3); };
    auto desc = [&](const unsigned char* base, int t) {
        const long t0 = kbeg + (long)t * kF32BlockKeys;
        const long left = kend - t0;
        // tiles at or past the end (the loop's trailing copies) cover no rows
        const long rows = left <= 0 ? 0 : (left < kF32BlockKeys ? left : kF32BlockKeys);
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(base + t0 * row_bytes),
                                                 (short)0, (int)(rows * row_bytes), kBufFlags);
    };
    // KVMap entries of this lane's 4 copy rows of tile t (-1 past the end)
    auto load_entries = [&](int t, long (&m)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long j = kbeg + (long)t * kF32BlockKeys + cp_row(i);
            m[i] = j < kend ? map[j] : -1L;
        }
    };
    long mcur[4] = {-1L, -1L, -1L, -1L};
    long mnext[4] = {-1L, -1L, -1L, -1L};
    __amdgpu_buffer_rsrc_t krs, vrs;
    unsigned kdst = 0, vdst = 0;
    auto prep_tile = [&](int t, unsigned char* kd, unsigned char* vd) {
        krs = desc(Kb, t);
        vrs = desc(Vb, t);
        kdst = (unsigned)__builtin_amdgcn_readfirstlane((int)(uintptr_t)kd) + 4096u * wave;
        vdst = (unsigned)__builtin_amdgcn_readfirstlane((int)(uintptr_t)vd) + 4096u * wave;
    };
    auto copy = [&](int i) {
        KVP_LDS void* kd = (KVP_LDS void*)(uintptr_t)(kdst + 1024u * i);
        KVP_LDS void* vd = (KVP_LDS void*)(uintptr_t)(vdst + 1024u * i);
        const int kc = k_chunk(i), vc = v_chunk(i);
        if (kMap && mcur[i] >= 0) {
            const unsigned char* ar = Ab + mcur[i] * 2 * row_bytes + hoff_b;
            __builtin_amdgcn_global_load_lds(ar + 16 * kc, kd, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(ar + row_bytes + 16 * vc, vd, 16, 0, 0);
        } else {
            const unsigned ro = (unsigned)cp_row(i) * rb + (unsigned)hoff_b;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, kd, 16, ro + 16u * kc, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, vd, 16, ro + 16u * vc, 0, 0, 0);
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[nb][v] = 0.f;
    float m_run = -INFINITY;
    float l_run = 0.f;
    const float cl2 = a.scale_log2;
    const unsigned kswz = (unsigned)(lq & 15);

    if (ntiles > 0) {
        if constexpr (kMap) {
            load_entries(0, mcur);
            load_entries(1, mnext);
        }
        prep_tile(0, k_lds0, v_lds0);
#pragma unroll
        for (int i = 0; i < 4; ++i) copy(i);
    }
    for (int t = 0; t < ntiles; ++t) {
        unsigned char* kcur = (t & 1) ? k_lds1 : k_lds0;
        unsigned char* vcur = (t & 1) ? v_lds1 : v_lds0;
        // every copy of tile t (and the entries of tile t+1) has landed; the
        // barrier publishes the tile and closes the reads of the other stage
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __syncthreads();
        if constexpr (kMap) {
#pragma unroll
            for (int i = 0; i < 4; ++i) mcur[i] = mnext[i];
            load_entries(t + 2, mnext);
        }
        prep_tile(t + 1, (t & 1) ? k_lds0 : k_lds1, (t & 1) ? v_lds0 : v_lds1);
        if (!active) {
#pragma unroll
            for (int i = 0; i < 4; ++i) copy(i);
            continue;
        }

        // S^T = K Q^T: 16 ds_read_b128 of K (row lq, logical chunk 2j + hh),
        // each read two k-steps ahead of its 4 MFMAs
        const unsigned kbase = (unsigned)(uintptr_t)kcur + (unsigned)(lq * 512);
        auto kaddr = [&](int j) {
            return kbase + 256u * (unsigned)(j >> 3) +
                   ((((unsigned)(2 * (j & 7) + hh)) ^ kswz) << 4);
        };
        f32x16 st;
#pragma unroll
        for (int v = 0; v < 16; ++v) st[v] = 0.f;
        u32x4 kr[3];
        kr[0] = lds_b128<0>(kaddr(0));
        kr[1] = lds_b128<0>(kaddr(1));
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            u32x4& ka = kr[j % 3];
            if (j + 1 < 16)
                lgkm_wait_keep1(ka);
            else
                lgkm_wait1x4(ka);
            if (j + 2 < 16) kr[(j + 2) % 3] = lds_b128<0>(kaddr(j + 2));
            const f32x4 kf = __builtin_bit_cast(f32x4, ka);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                st = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[i], qf[j][i], st, 0, 0, 0);
            if ((j & 3) == 3) copy(j >> 2);
        }

        float s[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) s[v] = st[v];
        const long t0 = kbeg + (long)t * kF32BlockKeys;
        if (t0 + kF32BlockKeys > kend) {
            const int lim = (int)(kend - t0) - 4 * hh;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int kc = 8 * (v >> 2) + (v & 3);
                if (kc >= lim) s[v] = -INFINITY;
            }
        }
        float p[16];
        auto exp_tile = [&](float mref) {
            float ra = 0.f, rb2 = 0.f;
#pragma unroll
            for (int v = 0; v < 16; v += 2) {
                p[v] = fast_exp2(fmaf(s[v], cl2, -mref));
                p[v + 1] = fast_exp2(fmaf(s[v + 1], cl2, -mref));
                ra += p[v];
                rb2 += p[v + 1];
            }
            const float rs = ra + rb2;
            return rs + other_half(rs);
        };
        float tot = exp_tile(m_run);
        if (__builtin_amdgcn_ballot_w64(!(tot <= kF32RowSumLimit))) {
            float mx = s[0];
#pragma unroll
            for (int v = 1; v < 16; ++v) mx = fmaxf(mx, s[v]);
            mx = fmaxf(mx, other_half(mx));
            const float m_new = fmaxf(m_run, mx * cl2);
            const float corr = fast_exp2(m_run - m_new);  // 0 while m_run is -inf
            l_run *= corr;
#pragma unroll
            for (int nb = 0; nb < 4; ++nb)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[nb][v] *= corr;
            m_run = m_new;
            tot = exp_tile(m_run);
        }
        l_run += tot;

        // O^T += V^T P^T: lane reads V[key][32 nb + lq] for its keys
        // 4*hh + 8*(v/4) + v%4 (row offsets are immediates); the V swizzle
        // bit of those rows is hh. A block's 16 reads go out while the
        // previous block's MFMAs run.
        const unsigned vbase = (unsigned)(uintptr_t)vcur + (unsigned)(4 * hh * 512 + 4 * (lq & 3));
        auto read_vb = [&](unsigned (&d)[16], int nb) {
            const unsigned ad = vbase + 16u * (unsigned)((8 * nb + (lq >> 2)) ^ (8 * hh));
            d[0] = lds_b32<0 * 512>(ad);
            d[1] = lds_b32<1 * 512>(ad);
            d[2] = lds_b32<2 * 512>(ad);
            d[3] = lds_b32<3 * 512>(ad);
            d[4] = lds_b32<8 * 512>(ad);
            d[5] = lds_b32<9 * 512>(ad);
            d[6] = lds_b32<10 * 512>(ad);
            d[7] = lds_b32<11 * 512>(ad);
            d[8] = lds_b32<16 * 512>(ad);
            d[9] = lds_b32<17 * 512>(ad);
            d[10] = lds_b32<18 * 512>(ad);
            d[11] = lds_b32<19 * 512>(ad);
            d[12] = lds_b32<24 * 512>(ad);
            d[13] = lds_b32<25 * 512>(ad);
            d[14] = lds_b32<26 * 512>(ad);
            d[15] = lds_b32<27 * 512>(ad);
        };
        unsigned vv[2][16];
        read_vb(vv[0], 0);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            unsigned (&cur)[16] = vv[nb & 1];
            lgkm_wait16(cur);
            if (nb < 3) read_vb(vv[(nb + 1) & 1], nb + 1);
#pragma unroll
            for (int v = 0; v < 16; ++v)
                o[nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(cur[v]), p[v], o[nb],
                                                              0, 0, 0);
        }
    }
    // the trailing copies land before the workgroup's LDS is released
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    if (!active) return;
    store_rows_f32(a, c, q, hh, o, m_run, l_run);
}

// ---------------------------------------------------------------------------
// split combine: out[q, h, :] = sum_s w_s O_s / sum_s w_s, w_s = 2^(lse_s - M)
// One thread per 8 output columns of one query row; every load of all splits
// is issued before any arithmetic (MAXS bounds the unrolled split loop).
// ---------------------------------------------------------------------------
template <typename OutT, int MAXS>
__device__ __forceinline__ void combine_block(const AttnArgs& a, long block) {
    const long gid = block * 256 + threadIdx.x;
    const int cols8 = a.D / 8;
    const long total = (long)a.frames * a.nq * cols8;
    if (gid >= total) return;
    const int c8 = (int)(gid % cols8);
    const long rq = gid / cols8;
    const int q = (int)(rq % a.nq);
    const int frame = (int)(rq / a.nq);
    const int head = (8 * c8) / kHeadDim;

    float lse[MAXS], pe[MAXS];
    f32x4 p0[MAXS], p1[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
        if (s < a.splits) {
            const long slab = (long)s * a.frames + frame;
            const long li = (slab * a.heads + head) * (long)a.nq + q;
            lse[s] = a.part_lse[li];
            pe[s] = sizeof(OutT) == 4 ? 0.f : a.part_exp[li];
            const long pofs = (slab * a.nq + q) * (long)a.D + 8 * c8;
            if constexpr (sizeof(OutT) == 4) {
                const float* po = static_cast<const float*>(a.part_o) + pofs;
                p0[s] = *reinterpret_cast<const f32x4*>(po);
                p1[s] = *reinterpret_cast<const f32x4*>(po + 4);
            } else {
                typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
                const f16x8 h =
                    *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(a.part_o) + pofs);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    p0[s][i] = (float)h[i];
                    p1[s][i] = (float)h[4 + i];
                }
            }
        }
    }
    // Partial s holds P_s * 2^e_s. With e0 = min_s e_s the result is
    // 2^-e0 * sum_s w_s 2^(e0 - e_s) (P_s 2^e_s) / sum_s w_s: every factor
    // 2^(e0 - e_s) <= 1, and 2^-e0 is applied once at the end.
    float mx = lse[0], e0 = pe[0];
#pragma unroll
    for (int s = 1; s < MAXS; ++s)
        if (s < a.splits) {
            mx = fmaxf(mx, lse[s]);
            e0 = fminf(e0, pe[s]);
        }
    float wsum = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
        if (s < a.splits) {
            const float w = fast_exp2(lse[s] - mx);
            wsum += w;
            const float ws = __builtin_amdgcn_ldexpf(w, (int)(e0 - pe[s]));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[i] = fmaf(ws, p0[s][i], acc[i]);
                acc[4 + i] = fmaf(ws, p1[s][i], acc[4 + i]);
            }
        }
    }
    const float inv = __builtin_amdgcn_ldexpf(1.0f / wsum, -(int)e0);
    OutT* out = reinterpret_cast<OutT*>(a.out) + (long)frame * a.q_fstride + (long)q * a.D + 8 * c8;
    if constexpr (sizeof(OutT) == 4) {
        const f32x4 w0 = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        const f32x4 w1 = {acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
        *reinterpret_cast<f32x4*>(out) = w0;
        *reinterpret_cast<f32x4*>(out + 4) = w1;
    } else {
        bf16x8 w;
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = (__bf16)(acc[i] * inv);
        *reinterpret_cast<bf16x8*>(out) = w;
    }
}

template <typename OutT, int MAXS>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
    combine_block<OutT, MAXS>(a, blockIdx.x);
}

template <typename OutT>
void launch_combine(const AttnArgs& a, hipStream_t st) {
    const long total = (long)a.frames * a.nq * (a.D / 8);
    const dim3 grid((unsigned)((total + 255) / 256));
    const dim3 block(256);
    if (a.splits <= 2)
        hipLaunchKernelGGL((attn_combine_kernel<OutT, 2>), grid, block, 0, st, a);
    else if (a.splits <= 4)
        hipLaunchKernelGGL((attn_combine_kernel<OutT, 4>), grid, block, 0, st, a);
    else if (a.splits <= 8)
        hipLaunchKernelGGL((attn_combine_kernel<OutT, 8>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((attn_combine_kernel<OutT, 16>), grid, block, 0, st, a);
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
// Split-partial workspace, one buffer per (device, stream): launches on one
// stream reuse its buffer in stream order, launches on different streams
// never share one. hipStreamPerThread is one handle value for every thread
// but a different stream in each, so its buffers are also keyed by thread.
// At most kMaxWorkspaces buffers per device are kept: a launch on another
// stream frees the least recently used one first (hipFree waits for the
// device, so no launch still reads it); kvp_attn_workspace_release frees a
// stream's buffer at once.
constexpr int kMaxWorkspaces = 8;
struct Workspace {
    int dev = -1;
    void* stream = nullptr;
    std::thread::id tid;  // hipStreamPerThread only
    void* ptr = nullptr;
    size_t bytes = 0;
    unsigned long use = 0;  // last use, for the eviction order
};
std::vector<Workspace> g_ws;
unsigned long g_ws_clock = 0;

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
                &nb, attn_fwd_bf16_kernel<__bf16, true, false, false>, kThreads, 0) == hipSuccess &&
            nb > 0)
            di.wg_per_cu_bf16 = nb;
        nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, attn_fwd_f32_kernel<true>, kThreads, 0) == hipSuccess && nb > 0)
            di.wg_per_cu_f32 = nb;
        di.ok = true;
    }
    return di;
}

std::thread::id stream_thread(void* stream) {
    return stream == static_cast<void*>(hipStreamPerThread) ? std::this_thread::get_id()
                                                            : std::thread::id();
}

// Caller holds g_mu.
void free_workspace_at(size_t i) {
    if (g_ws[i].ptr) (void)hipFree(g_ws[i].ptr);
    g_ws.erase(g_ws.begin() + (long)i);
}

void* workspace(int dev, void* stream, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    const std::thread::id tid = stream_thread(stream);
    long found = -1, n_dev = 0, lru = -1;
    for (size_t i = 0; i < g_ws.size(); ++i) {
        if (g_ws[i].dev != dev) continue;
        ++n_dev;
        if (g_ws[i].stream == stream && g_ws[i].tid == tid) found = (long)i;
        if (lru < 0 || g_ws[i].use < g_ws[(size_t)lru].use) lru = (long)i;
    }
    if (found < 0) {
        if (n_dev >= kMaxWorkspaces) free_workspace_at((size_t)lru);
        g_ws.push_back(Workspace{dev, stream, tid, nullptr, 0, 0});
        found = (long)g_ws.size() - 1;
    }
    Workspace& w = g_ws[(size_t)found];
    w.use = ++g_ws_clock;
    if (w.bytes < bytes) {
        // Growing waits for the in-flight users of the old buffer: launches
        // on this same stream.
        if (w.ptr) {
            (void)hipStreamSynchronize(static_cast<hipStream_t>(stream));
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
// workgroups. Splitting divides the per-workgroup key loop but every split
// writes and the combine re-reads one fp32 partial of the whole output
// (about one tile-round of time per split at the C3 shape, measured), plus a
// fixed cost for the extra launch.
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
        if (s > 1) t += 2.0 + 1.2 * (double)s * (double)base_wg / 156.0;
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

// Positional form used by the reference-signature entry points: every frame
// attends the same key range.
int launch_attention(int dtype, const void* q, const void* k, const void* v, const void* arena,
                     const long* kvmap, void* out, int nq, int D, int heads, int frames,
                     long q_fstride, long kv_fstride, long map_fstride, long key_begin,
                     long key_end, void* stream) {
    AttnLaunch L;
    L.dtype = dtype;
    L.q = q;
    L.k = k;
    L.v = v;
    L.arena = arena;
    L.kvmap = kvmap;
    L.out = out;
    L.nq = nq;
    L.D = D;
    L.heads = heads;
    L.frames = frames;
    L.q_fstride = q_fstride;
    L.kv_fstride = kv_fstride;
    L.map_fstride = map_fstride;
    L.key_begin = key_begin;
    L.key_end = key_end;
    L.stream = stream;
    return launch_attention(L);
}

namespace {

constexpr long kNoSpanLimit = 0x4000000000000000L;

// Argument checks that need no device. Returns 0 or 1 with the error recorded.
int validate_launch(const AttnLaunch& L) {
    if (L.dtype != 0 && L.dtype != 1) {
        set_error("attention: dtype %d not supported (0 = fp32, 1 = bf16)", L.dtype);
        return 1;
    }
    if (L.heads <= 0 || L.D != L.heads * kHeadDim) {
        set_error("attention: head_dim must be 128 (D=%d heads=%d)", L.D, L.heads);
        return 1;
    }
    if (L.nq <= 0 || L.frames <= 0) {
        set_error("attention: empty launch (nq=%d frames=%d)", L.nq, L.frames);
        return 1;
    }
    if (L.key_end <= L.key_begin || L.key_begin < 0) {
        set_error("attention: empty or negative key range [%ld, %ld)", L.key_begin, L.key_end);
        return 1;
    }
    if (L.kend_step < 0 || L.q_fstride < 0 || L.kv_fstride < 0 || L.map_fstride < 0 ||
        L.arena_fstride < 0) {
        set_error("attention: negative frame stride");
        return 1;
    }
    if (L.kend_step != 0 && !L.layer && L.frames > 1) {
        set_error("attention: per-frame key ranges need a layer launch");
        return 1;
    }
    if (!L.q || !L.k || !L.v || !L.out) {
        set_error("attention: null q/k/v/out pointer");
        return 1;
    }
    const long last = (long)(L.frames - 1);
    const long max_key_end = L.key_end + last * L.kend_step;
    if (max_key_end > 0x7fffffffL ||
        last * L.kv_fstride / L.D + max_key_end > 0x7fffffffL) {
        set_error("attention: key rows must stay below 2^31");
        return 1;
    }
    if (L.kvmap && !L.arena) {
        set_error("attention: kvmap given without arena");
        return 1;
    }
    if (L.gdesc && (!L.kvmap || L.dtype != 1 || L.cold_rows_nt || L.gd_fstride < 0 ||
                    (uintptr_t)L.gdesc % 8)) {
        set_error("attention: group descriptors need a bf16 KVMap launch without the "
                  "non-temporal lever, an 8-byte aligned table and a non-negative stride");
        return 1;
    }
    if (L.arena_fstride % 16) {
        set_error("attention: arena regions must be 16-byte aligned");
        return 1;
    }
    if (((uintptr_t)L.q | (uintptr_t)L.k | (uintptr_t)L.v | (uintptr_t)L.out |
         (uintptr_t)L.arena) % 16) {
        set_error("attention: q/k/v/out/arena must be 16-byte aligned");
        return 1;
    }
    return 0;
}

// Fills the kernel arguments and the launch shape of a validated launch.
int prepare_launch(const AttnLaunch& L, const DeviceInfo& di, AttnArgs& a, LaunchPlan& p) {
    const long max_key_end = L.key_end + (long)(L.frames - 1) * L.kend_step;
    const long max_span = L.max_span > 0 ? L.max_span : kNoSpanLimit;
    // longest range of any frame: the last frame's (ranges only grow)
    long span_last = max_key_end - L.key_begin;
    if (span_last > max_span) span_last = max_span;

    const int bk = L.dtype == 1 ? kBf16BlockKeys : kF32BlockKeys;
    // A one-frame layer is an ordinary launch: it may then split its key
    // range when its workgroups underfill the GPU.
    const bool layer = L.layer && L.frames > 1;
    if (layer) {
        p.nqb = (L.nq + kBlockQ - 1) / kBlockQ;
        p.splits = 1;
        p.keys_per_split = ((span_last + bk - 1) / bk) * bk;
        const long cols = (long)L.heads * p.nqb;
        p.grid = (long)kNumXcd * ((cols + kNumXcd - 1) / kNumXcd) * L.frames;
    } else {
        p = plan_launch(L.dtype, L.nq, L.heads, L.frames, span_last, di);
    }
    if (p.grid > 0x7fffffffL) {
        set_error("attention: grid too large");
        return 1;
    }
    // every frame's table (gd_fstride entries, also for one frame) covers
    // the 16-row groups of the longest range
    if (L.gdesc &&
        L.gd_fstride < 4 * ((span_last + kBf16BlockKeys - 1) / kBf16BlockKeys)) {
        set_error("attention: group-descriptor stride %ld below the %ld groups of a range",
                  L.gd_fstride, 4 * ((span_last + kBf16BlockKeys - 1) / kBf16BlockKeys));
        return 1;
    }

    a.q = L.q;
    a.k = L.k;
    a.v = L.v;
    a.arena = L.arena;
    a.kvmap = L.kvmap;
    a.gdesc = L.gdesc;
    a.gd_fstride = L.gd_fstride;
    a.out = L.out;
    a.part_o = nullptr;
    a.part_lse = nullptr;
    a.part_exp = nullptr;
    a.q_fstride = L.q_fstride;
    a.kv_fstride = L.kv_fstride;
    a.map_fstride = L.map_fstride;
    a.arena_fstride = L.arena_fstride;
    a.key_begin = L.key_begin;
    a.key_end = L.key_end;
    a.kend_step = L.kend_step;
    a.max_span = max_span;
    a.keys_per_split = p.keys_per_split;
    a.nq = L.nq;
    a.D = L.D;
    a.heads = L.heads;
    a.frames = L.frames;
    a.splits = p.splits;
    a.nqb = p.nqb;
    a.layer_order = layer ? 1 : 0;
    // Only the bf16 kernel orders its walks (the fp32 kernel walks every
    // range upward); the count assumes the occupancy the kernel was
    // measured at, and only steers the order, never correctness.
    a.xcd_slots = layer && L.dtype == 1 ? std::max(1, di.cus / kNumXcd) * di.wg_per_cu_bf16 : 0;
    a.cyclic = max_key_end - L.key_begin > max_span ? 1 : 0;
    a.scale_log2 = kLog2e / sqrtf((float)kHeadDim);
    return 0;
}

// Workspace of a split launch: partial rows, then the log-sum-exps, then the
// row-scale exponents, each 256-byte aligned.
size_t partial_bytes(const AttnArgs& a, int dtype, size_t* lse_offset, size_t* exp_offset) {
    const size_t po = (size_t)a.splits * a.frames * a.nq * a.D * (dtype == 1 ? 2 : 4);
    const size_t pl = (size_t)a.splits * a.frames * a.heads * a.nq * sizeof(float);
    const size_t off = ((po + 255) / 256) * 256;
    const size_t off2 = off + ((pl + 255) / 256) * 256;
    if (lse_offset) *lse_offset = off;
    if (exp_offset) *exp_offset = off2;
    return off2 + pl;
}

}  // namespace

size_t attention_workspace_bytes(const AttnLaunch& L) {
    if (validate_launch(L)) return 0;
    const int dev = current_device();
    if (dev < 0) return 0;
    AttnArgs a;
    LaunchPlan p;
    if (prepare_launch(L, device_info(dev), a, p)) return 0;
    return p.splits > 1 ? partial_bytes(a, L.dtype, nullptr, nullptr) : 0;
}

// Core launcher shared by all public attention entry points.
int launch_attention(const AttnLaunch& L) {
    if (validate_launch(L)) return 1;
    const int dev = current_device();
    if (dev < 0) {
        set_error("attention: no HIP device available");
        return 1;
    }
    const DeviceInfo di = device_info(dev);
    AttnArgs a;
    LaunchPlan p;
    if (prepare_launch(L, di, a, p)) return 1;

    if (p.splits > 1) {
        size_t lse_off = 0, exp_off = 0;
        const size_t need = partial_bytes(a, L.dtype, &lse_off, &exp_off);
        char* ws = nullptr;
        if (L.workspace) {
            if (L.workspace_bytes < need) {
                set_error("attention: this launch needs %zu bytes of split partials, above the "
                          "%zu-byte workspace it was given",
                          need, L.workspace_bytes);
                return 1;
            }
            ws = static_cast<char*>(L.workspace);
        } else {
            ws = static_cast<char*>(workspace(dev, L.stream, need));
            if (!ws) {
                set_error("attention: workspace allocation of %zu bytes failed", need);
                return 1;
            }
        }
        a.part_o = ws;
        a.part_lse = reinterpret_cast<float*>(ws + lse_off);
        a.part_exp = reinterpret_cast<float*>(ws + exp_off);
    }
    hipStream_t st = static_cast<hipStream_t>(L.stream);
    if (L.dtype == 1) {
        // the non-temporal lever walks every range upward or reversed
        if (a.kvmap && L.cold_rows_nt)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<__bf16, true, true, false>),
                               dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
        else if (a.gdesc && a.cyclic)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<__bf16, true, false, true, true>),
                               dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
        else if (a.gdesc)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<__bf16, true, false, false, true>),
                               dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
        else if (a.kvmap && a.cyclic)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<__bf16, true, false, true>),
                               dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
        else if (a.kvmap)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<__bf16, true, false, false>),
                               dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
        else if (a.cyclic)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<__bf16, false, false, true>),
                               dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
        else
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<__bf16, false, false, false>),
                               dim3((unsigned)p.grid), dim3(kThreads), 0, st, a);
    } else {
        if (a.kvmap)
            hipLaunchKernelGGL(attn_fwd_f32_kernel<true>, dim3((unsigned)p.grid), dim3(kThreads), 0,
                               st, a);
        else
            hipLaunchKernelGGL(attn_fwd_f32_kernel<false>, dim3((unsigned)p.grid), dim3(kThreads), 0,
                               st, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("attention launch: %s", hipGetErrorString(e));
        return 1;
    }
    if (p.splits > 1) {
        if (L.dtype == 1)
            launch_combine<__bf16>(a, st);
        else
            launch_combine<float>(a, st);
        e = hipGetLastError();
        if (e != hipSuccess) {
            set_error("attention combine launch: %s", hipGetErrorString(e));
            return 1;
        }
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Allocation-free attention (kvp_attn_forward_range_noalloc): the split
// partials of a launch go to `scratch`, a fixed device array of this code
// object, instead of the per-(device, stream) workspace. Every GPU the library
// runs on holds its own copy from module load until the process ends. Host
// code never passes the array's name to a kernel (on the host it is only a
// stand-in for the symbol): the device address is looked up once per device
// with hipGetSymbolAddress, with that device current, and that address is
// what the kernels receive. Nothing in the array has to start at zero: the
// attention kernel writes every partial row, log-sum-exp and row-scale
// exponent the combine then reads. All calls on one GPU share the array, so
// calls that overlap on one GPU (two streams, two threads) race.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // per device; null until looked up

void* scratch_address(int dev) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_error("attention scratch: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}
}  // namespace

int launch_attention_noalloc(AttnLaunch L) {
    if (validate_launch(L)) return 1;
    const int dev = current_device();
    if (dev < 0) {
        set_error("attention: no HIP device available");
        return 1;
    }
    void* ptr = scratch_address(dev);
    if (!ptr) return 1;
    L.workspace = ptr;
    L.workspace_bytes = kScratchBytes;
    return launch_attention(L);
}

int attention_splits(int dtype, int nq, int heads, int frames, long span) {
    if (nq <= 0 || heads <= 0 || frames <= 0 || span <= 0) return 0;
    DeviceInfo di;
    const int dev = current_device();
    if (dev >= 0) di = device_info(dev);
    return plan_launch(dtype, nq, heads, frames, span, di).splits;
}

}  // namespace kvp

extern "C" int kvp_attn_workspace_release(void* stream) {
    const int dev = kvp::current_device();
    if (dev < 0) return 1;
    (void)hipStreamSynchronize(static_cast<hipStream_t>(stream));
    std::lock_guard<std::mutex> lk(kvp::g_mu);
    const std::thread::id tid = kvp::stream_thread(stream);
    for (size_t i = 0; i < kvp::g_ws.size(); ++i) {
        if (kvp::g_ws[i].dev == dev && kvp::g_ws[i].stream == stream && kvp::g_ws[i].tid == tid) {
            kvp::free_workspace_at(i);
            break;
        }
    }
    return 0;
}

extern "C" long kvp_attn_workspace_count(void) {
    std::lock_guard<std::mutex> lk(kvp::g_mu);
    return (long)kvp::g_ws.size();
}

extern "C" int kvp_attn_block_queries(int) { return kvp::kBlockQ; }
extern "C" int kvp_attn_block_keys(int dtype) {
    return dtype == 1 ? kvp::kBf16BlockKeys : kvp::kF32BlockKeys;
}
extern "C" int kvp_attn_splits(int dtype, int nq, int heads, int frames, long span) {
    return kvp::attention_splits(dtype, nq, heads, frames, span);
}

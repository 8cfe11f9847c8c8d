// Upstream motion producer of the KV-arena path, gfx950-native: dense
// Farneback optical flow between consecutive gray frames and the per-tile
// change rates the gating policies rank (reference:
// traces/gen_motion_from_video.py:104-135, which calls OpenCV's
// cv2.calcOpticalFlowFarneback with pyr_scale 0.5, levels 3, winsize 15,
// iterations 3, poly_n 5, poly_sigma 1.2, flags 0).
//
// The algorithm is the one OpenCV 4.x publishes (modules/video/src/
// optflowgf.cpp; Farneback, "Two-frame motion estimation based on
// polynomial expansion", SCIA 2003), laid out for the GPU: every kernel
// covers all frames (or all consecutive pairs) of a clip in one launch, and
// each frame's pyramid image and polynomial expansion are computed once per
// level and shared by the two pairs that use it.
//
//   blur_rows_kernel         Gaussian pre-blur, horizontal pass, reflect-101
//                            border, uint8 -> fp32: one source row per
//                            workgroup staged in LDS, computed only at the
//                            columns the level's resize samples.
//   blur_cols_resize_kernel  vertical pass fused with the bilinear resize to
//                            the level size (half-pixel centres, clamped
//                            edges): only the 2 x 2 samples each level pixel
//                            needs are blurred.
//   poly_exp_kernel          quadratic fit under a separable Gaussian
//                            applicability (2n+1 taps), replicated border;
//                            64 x 16 tile + halo in LDS, vertical then
//                            horizontal pass; 5 fp32 planes
//                            [b_y, b_x, a_yy, a_xx, a_xy].
//   update_matrices_kernel   per pixel: the next frame's expansion sampled
//                            bilinearly at x + flow, averaged with the
//                            previous frame's, border down-weighting, and the
//                            5 values of A^T A and A^T delta-b. Its first
//                            call per level also produces the initial flow
//                            (zero, or the coarser level's flow resized and
//                            scaled by 1/pyr_scale).
//   update_flow_kernel       winsize x winsize box average of those 5 planes
//                            (replicated border): fp64 running column sums
//                            slid down a strip of rows, parked in LDS 4 rows
//                            at a time, sliding sums along runs of 2 columns;
//                            then the regularised 2 x 2 solve in fp64.
//   update_flow_ring_kernel  the same for winsize 15 (the reference's), with
//                            each column's 15 window rows held in a register
//                            ring, so that M is read once instead of twice,
//                            and the next rows' loads in flight across each
//                            horizontal pass.
//   flow_cells_kernel        |flow| averaged over grid cells (one workgroup
//                            per cell row), then tile_change_kernel: the mean
//                            of each run of tile_tokens cells in fp64.
//
// Layout in HBM: frames uint8 [n, H, W] (any frame stride); pyramid image
// fp32 [n, h, w]; expansion fp32 [n][5][h*w]; matrices fp32 [pairs][5][h*w];
// flow fp32 [pairs, h, w, 2] (x, y), the final level written straight into
// the caller's output.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <vector>

#include "kvp_internal.h"
#include "kvp_motion.h"

namespace kvp {
namespace {

constexpr int kMaxBlurTaps = 127;   // pre-blur kernel size (level scale >= 1/26)
constexpr int kMaxPolyN = 8;        // applicability half-width
constexpr int kMaxBoxHalf = 24;     // winsize <= 49
constexpr int kMinLevelSide = 32;   // OpenCV's min_size for a pyramid level
constexpr int kBorder = 5;          // down-weighted border width
constexpr int kMinSide = 2 * kBorder;
constexpr int kMaxSide = 8192;
constexpr int kMaxFrames = 4096;
constexpr int kPeTileW = 64, kPeTileH = 16;
constexpr int kBfBatch = 4;       // box filter: rows parked in LDS at a time
constexpr int kBfRun = 2;         // box filter: output columns per sliding run
constexpr int kBfTargetGroups = 2048;
// register-ring box filter (update_flow_ring_kernel): window half-width it
// serves (winsize 15), rows per workgroup bounds, target workgroups per launch
constexpr int kBfRingHalf = 7;
constexpr int kBfRingRows = 45;
constexpr int kBfRingMinRows = 10;
constexpr int kBfRingGroups = 1024;

struct BlurTaps {
    int ksize;
    float k[kMaxBlurTaps];
};

struct PolyTaps {
    int n;
    float g[2 * kMaxPolyN + 1];
    float xg[2 * kMaxPolyN + 1];
    float xxg[2 * kMaxPolyN + 1];
    double ig11, ig03, ig33, ig55;
};

__device__ __forceinline__ int reflect101(int i, int n) {
    if (n == 1) return 0;
    const int period = 2 * n - 2;
    i = i < 0 ? -i : i;
    i %= period;
    return i >= n ? period - i : i;
}

// resize INTER_LINEAR source taps of destination index d: s0, s1 and the
// weight of s1 (OpenCV: fx = (d + 0.5) * scale - 0.5, clamped at both ends).
__device__ __forceinline__ void linear_tap(int d, double scale, int src, int& s0, int& s1,
                                           float& w) {
    float f = (float)((d + 0.5) * scale - 0.5);
    int s = (int)floorf(f);
    f -= (float)s;
    if (s < 0) { f = 0.f; s = 0; }
    if (s >= src - 1) { f = 0.f; s = src - 1; }
    s0 = s;
    s1 = min(s + 1, src - 1);
    w = f;
}

// Horizontal pre-blur pass of one source row per workgroup, computed only at
// the columns the level's resize samples: column j of the compact output is
// source column tap(j / 2) + (j & 1) (both bilinear taps of level column
// j / 2), or every column when the level has the source size. The row and its
// reflect-101 halo are staged in LDS once.
__global__ __launch_bounds__(256) void blur_rows_kernel(const uint8_t* __restrict__ src,
                                                        long frame_stride, int W, int H,
                                                        float* __restrict__ out, int ncols,
                                                        int same_size, double sx_scale,
                                                        BlurTaps t) {
    extern __shared__ float row[];
    const int f = blockIdx.z, y = blockIdx.x;
    const uint8_t* s = src + (long)f * frame_stride + (long)y * W;
    const int h = t.ksize / 2;
    float* r = row + h;                      // r[-h .. W + h)
    if ((W & 3) == 0 && (((uintptr_t)s) & 3) == 0) {
        const uchar4* s4 = reinterpret_cast<const uchar4*>(s);
        for (int i = threadIdx.x; i < W / 4; i += 256) {
            const uchar4 v = s4[i];
            r[4 * i] = v.x;
            r[4 * i + 1] = v.y;
            r[4 * i + 2] = v.z;
            r[4 * i + 3] = v.w;
        }
    } else {
        for (int i = threadIdx.x; i < W; i += 256) r[i] = s[i];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 2 * h; i += 256) {
        const int c = i < h ? i - h : W + (i - h);       // halo columns
        r[c] = r[reflect101(c, W)];
    }
    __syncthreads();
    float* o = out + ((long)f * H + y) * ncols;
    for (int j = threadIdx.x; j < ncols; j += 256) {
        int c;
        if (same_size) {
            c = j;
        } else {
            int c0, c1;
            float wt;
            linear_tap(j >> 1, sx_scale, W, c0, c1, wt);
            c = (j & 1) ? c1 : c0;
        }
        float acc = 0.f;
        for (int k = 0; k < t.ksize; ++k) acc += t.k[k] * r[c - h + k];
        o[j] = acc;
    }
}

// Vertical pre-blur pass fused with the bilinear resize: level pixel (x, y)
// blends the vertically blurred compact columns 2x, 2x + 1 (or x at the
// source size) at the two source rows its resize taps name.
__global__ __launch_bounds__(256) void blur_cols_resize_kernel(
        const float* __restrict__ hb, int ncols, int W, int H, float* __restrict__ out, int w,
        int h, double sx_scale, double sy_scale, int same_size, BlurTaps t) {
    const int x = blockIdx.x * 64 + (threadIdx.x & 63);
    const int y = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int f = blockIdx.z;
    if (x >= w || y >= h) return;
    const float* base = hb + (long)f * H * ncols;
    const int hk = t.ksize / 2;
    auto col = [&](int r, int c) {
        float acc = 0.f;
        for (int j = 0; j < t.ksize; ++j)
            acc += t.k[j] * base[(long)reflect101(r - hk + j, H) * ncols + c];
        return acc;
    };
    float v;
    if (same_size) {
        v = col(y, x);
    } else {
        int xa, xb, ya, yb;
        float wx, wy;
        linear_tap(x, sx_scale, W, xa, xb, wx);
        linear_tap(y, sy_scale, H, ya, yb, wy);
        const float r0 = col(ya, 2 * x) * (1.f - wx) + col(ya, 2 * x + 1) * wx;
        const float r1 = col(yb, 2 * x) * (1.f - wx) + col(yb, 2 * x + 1) * wx;
        v = r0 * (1.f - wy) + r1 * wy;
    }
    out[(long)f * w * h + (long)y * w + x] = v;
}

__global__ __launch_bounds__(256) void poly_exp_kernel(const float* __restrict__ img, int w,
                                                       int h, float* __restrict__ R,
                                                       PolyTaps t) {
    constexpr int MW = kPeTileW + 2 * kMaxPolyN;
    constexpr int MH = kPeTileH + 2 * kMaxPolyN;
    __shared__ float src[MH * MW];
    __shared__ float vp[3][kPeTileH * MW];
    const int n = t.n;
    const int f = blockIdx.z;
    const int X0 = blockIdx.x * kPeTileW, Y0 = blockIdx.y * kPeTileH;
    const long P = (long)w * h;
    const float* I = img + (long)f * P;
    const int tw = kPeTileW + 2 * n, th = kPeTileH + 2 * n;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < th; r += 4) {
        const float* Ir = I + (long)min(max(Y0 - n + r, 0), h - 1) * w;
        for (int c = tx; c < tw; c += 64) src[r * MW + c] = Ir[min(max(X0 - n + c, 0), w - 1)];
    }
    __syncthreads();
    for (int r = ty; r < kPeTileH; r += 4)
    for (int c = tx; c < tw; c += 64) {
        float s0 = src[(r + n) * MW + c] * t.g[n], s1 = 0.f, s2 = 0.f;
        for (int k = 1; k <= n; ++k) {
            const float lo = src[(r + n - k) * MW + c], hi = src[(r + n + k) * MW + c];
            const float p = lo + hi;
            s0 += t.g[n + k] * p;
            s1 += t.xg[n + k] * (hi - lo);
            s2 += t.xxg[n + k] * p;
        }
        vp[0][r * MW + c] = s0;
        vp[1][r * MW + c] = s1;
        vp[2][r * MW + c] = s2;
    }
    __syncthreads();
    float* Rf = R + (long)f * 5 * P;
    for (int r = ty; r < kPeTileH; r += 4) {
        const int c = tx;
        const int x = X0 + c, y = Y0 + r;
        if (x >= w || y >= h) continue;
        const float* v0 = &vp[0][r * MW + c + n];
        const float* v1 = &vp[1][r * MW + c + n];
        const float* v2 = &vp[2][r * MW + c + n];
        const float g0 = t.g[n];
        float b1 = v0[0] * g0, b2 = 0.f, b3 = v1[0] * g0, b4 = 0.f, b5 = v2[0] * g0, b6 = 0.f;
        for (int k = 1; k <= n; ++k) {
            const float gk = t.g[n + k], xgk = t.xg[n + k], xxgk = t.xxg[n + k];
            const float tg = v0[k] + v0[-k];
            b1 += tg * gk;
            b4 += tg * xxgk;
            b2 += (v0[k] - v0[-k]) * xgk;
            b3 += (v1[k] + v1[-k]) * gk;
            b6 += (v1[k] - v1[-k]) * xgk;
            b5 += (v2[k] + v2[-k]) * gk;
        }
        const long o = (long)y * w + x;
        Rf[o] = (float)(b3 * t.ig11);
        Rf[P + o] = (float)(b2 * t.ig11);
        Rf[2 * P + o] = (float)(b1 * t.ig03 + b5 * t.ig33);
        Rf[3 * P + o] = (float)(b1 * t.ig03 + b4 * t.ig33);
        Rf[4 * P + o] = (float)(b6 * t.ig55);
    }
}

__device__ __forceinline__ float border_weight(int i) {
    return i == 0 || i == 1 ? 0.14f : 0.4472f;
}

// mode 0: read flow; 1: zero initial flow; 2: initial flow = the coarser
// level's flow (cw x ch) resized bilinearly, times flow_mul.
__global__ __launch_bounds__(256) void update_matrices_kernel(
        const float* __restrict__ R, int w, int h, float2* __restrict__ flow,
        float* __restrict__ M, int mode, const float2* __restrict__ coarse, int cw, int ch,
        double cx_scale, double cy_scale, float flow_mul, int write_flow) {
    const long P = (long)w * h;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const int p = blockIdx.y;
    if (i >= P) return;
    const int y = (int)(i / w), x = (int)(i - (long)y * w);
    float dx = 0.f, dy = 0.f;
    if (mode == 0) {
        const float2 d = flow[(long)p * P + i];
        dx = d.x;
        dy = d.y;
    } else if (mode == 2) {
        int xa, xb, ya, yb;
        float wx, wy;
        linear_tap(x, cx_scale, cw, xa, xb, wx);
        linear_tap(y, cy_scale, ch, ya, yb, wy);
        const float2* C = coarse + (long)p * cw * ch;
        const float2 a = C[(long)ya * cw + xa], b = C[(long)ya * cw + xb];
        const float2 c = C[(long)yb * cw + xa], d = C[(long)yb * cw + xb];
        const float rx0 = a.x * (1.f - wx) + b.x * wx, ry0 = a.y * (1.f - wx) + b.y * wx;
        const float rx1 = c.x * (1.f - wx) + d.x * wx, ry1 = c.y * (1.f - wx) + d.y * wx;
        dx = (rx0 * (1.f - wy) + rx1 * wy) * flow_mul;
        dy = (ry0 * (1.f - wy) + ry1 * wy) * flow_mul;
    }
    if (write_flow) flow[(long)p * P + i] = make_float2(dx, dy);

    const float* R0 = R + (long)p * 5 * P;
    const float* R1 = R0 + 5 * P;
    const float q0 = R0[i], q1 = R0[P + i], q2 = R0[2 * P + i], q3 = R0[3 * P + i],
                q4 = R0[4 * P + i];
    float fx = (float)x + dx, fy = (float)y + dy;
    // keep the float -> int conversion defined; anything this far out is outside
    fx = fminf(fmaxf(fx, -1e8f), 1e8f);
    fy = fminf(fmaxf(fy, -1e8f), 1e8f);
    const int x1 = (int)floorf(fx), y1 = (int)floorf(fy);
    fx -= (float)x1;
    fy -= (float)y1;
    float r2, r3, r4, r5, r6;
    if ((unsigned)x1 < (unsigned)(w - 1) && (unsigned)y1 < (unsigned)(h - 1)) {
        const float a00 = (1.f - fx) * (1.f - fy), a01 = fx * (1.f - fy);
        const float a10 = (1.f - fx) * fy, a11 = fx * fy;
        const long o = (long)y1 * w + x1;
        const float* s = R1 + o;
        r2 = a00 * s[0] + a01 * s[1] + a10 * s[w] + a11 * s[w + 1];
        s += P;
        r3 = a00 * s[0] + a01 * s[1] + a10 * s[w] + a11 * s[w + 1];
        s += P;
        r4 = a00 * s[0] + a01 * s[1] + a10 * s[w] + a11 * s[w + 1];
        s += P;
        r5 = a00 * s[0] + a01 * s[1] + a10 * s[w] + a11 * s[w + 1];
        s += P;
        r6 = a00 * s[0] + a01 * s[1] + a10 * s[w] + a11 * s[w + 1];
        r4 = (q2 + r4) * 0.5f;
        r5 = (q3 + r5) * 0.5f;
        r6 = (q4 + r6) * 0.25f;
    } else {
        r2 = r3 = 0.f;
        r4 = q2;
        r5 = q3;
        r6 = q4 * 0.5f;
    }
    r2 = (q0 - r2) * 0.5f;
    r3 = (q1 - r3) * 0.5f;
    r2 += r4 * dy + r6 * dx;
    r3 += r6 * dy + r5 * dx;
    if (x < kBorder || x >= w - kBorder || y < kBorder || y >= h - kBorder) {
        const float sc = (x < kBorder ? border_weight(x) : 1.f) *
                         (x >= w - kBorder ? border_weight(w - x - 1) : 1.f) *
                         (y < kBorder ? border_weight(y) : 1.f) *
                         (y >= h - kBorder ? border_weight(h - y - 1) : 1.f);
        r2 *= sc;
        r3 *= sc;
        r4 *= sc;
        r5 *= sc;
        r6 *= sc;
    }
    float* Mp = M + (long)p * 5 * P + i;
    Mp[0] = r4 * r4 + r6 * r6;
    Mp[P] = (r4 + r5) * r6;
    Mp[2 * P] = r5 * r5 + r6 * r6;
    Mp[3 * P] = r4 * r2 + r6 * r3;
    Mp[4 * P] = r6 * r2 + r5 * r3;
}

// One workgroup = a strip of COLS - 2m output columns (COLS loaded columns
// with the halo, one thread each) and `rows` output rows. Each thread keeps
// fp64 running vertical sums of the 5 planes for its column (the entering
// row added, the leaving row subtracted, replicated border) and parks them
// in LDS for kBfBatch rows at a time; then each thread turns a run of
// kBfRun columns of one parked row into box sums with a sliding horizontal
// sum and solves those pixels.
template <int COLS>
__global__ __launch_bounds__(COLS) void update_flow_kernel(const float* __restrict__ M, int w,
                                                           int h, int m, int rows, double scale,
                                                           float2* __restrict__ flow) {
    __shared__ float buf[kBfBatch][5][COLS];
    const int tw = COLS - 2 * m;
    const int X0 = blockIdx.x * tw;
    const int Y0 = blockIdx.y * rows;
    const int p = blockIdx.z;
    const long P = (long)w * h;
    const float* Mp = M + (long)p * 5 * P;
    float2* Fp = flow + (long)p * P;
    const int tid = threadIdx.x;
    const int xc = min(max(X0 - m + tid, 0), w - 1);
    double vs[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
    for (int r = Y0 - m; r <= Y0 + m; ++r) {
        const float* q = Mp + (long)min(max(r, 0), h - 1) * w + xc;
#pragma unroll
        for (int c = 0; c < 5; ++c) vs[c] += q[c * P];
    }
    const int yend = min(Y0 + rows, h);
    const int xend = min(tw, w - X0);                 // output columns of this strip
    const int runs = (xend + kBfRun - 1) / kBfRun;
    for (int yb = Y0; yb < yend; yb += kBfBatch) {
        const int nr = min(kBfBatch, yend - yb);
#pragma unroll
        for (int r = 0; r < kBfBatch; ++r) {
            if (r < nr) {
#pragma unroll
                for (int c = 0; c < 5; ++c) buf[r][c][tid] = (float)vs[c];
                const int y = yb + r;
                if (y + 1 < yend) {
                    const float* qa = Mp + (long)min(y + m + 1, h - 1) * w + xc;
                    const float* qs = Mp + (long)max(y - m, 0) * w + xc;
#pragma unroll
                    for (int c = 0; c < 5; ++c) vs[c] += (double)qa[c * P] - (double)qs[c * P];
                }
            }
        }
        __syncthreads();
        for (int j = tid; j < nr * runs; j += COLS) {
            const int r = j / runs;
            const int x0 = (j - r * runs) * kBfRun;
            const int n = min(kBfRun, xend - x0);
            float s[5][kBfRun];
#pragma unroll
            for (int c = 0; c < 5; ++c) {
                const float* v = &buf[r][c][x0];
                float a = 0.f;
                for (int k = 0; k <= 2 * m; ++k) a += v[k];
                s[c][0] = a;
#pragma unroll
                for (int i = 1; i < kBfRun; ++i) {
                    if (i < n) a += v[i + 2 * m] - v[i - 1];
                    s[c][i] = a;
                }
            }
            float2* out = Fp + (long)(yb + r) * w + X0 + x0;
#pragma unroll
            for (int i = 0; i < kBfRun; ++i) {
                if (i < n) {
                    const double g11 = s[0][i] * scale, g12 = s[1][i] * scale;
                    const double g22 = s[2][i] * scale, h1 = s[3][i] * scale;
                    const double h2 = s[4][i] * scale;
                    const double idet = 1.0 / (g11 * g22 - g12 * g12 + 1e-3);
                    out[i] = make_float2((float)((g11 * h2 - g12 * h1) * idet),
                                         (float)((g22 * h1 - g12 * h2) * idet));
                }
            }
        }
        __syncthreads();
    }
}

// The same box filter and solve for winsize 2*kM+1 with the window's rows
// kept in registers. update_flow_kernel reads every value of M twice (when
// its row enters a column's window and again when it leaves); here each
// thread keeps the 2kM+1 rows of its column's window for the 5 planes in a
// ring of registers, so the leaving row's values come from the ring and M is
// read once per strip (plus the first window of each workgroup's rows). The
// row loop is unrolled by the ring period, so every ring slot is a static
// register; rows are parked in LDS kRB at a time (kRB divides the period)
// for the horizontal pass. Only the first `ncols` threads load a column:
// the host sizes the strips to the level's width. The running sums see the
// same values in the same order as update_flow_kernel (fp64: entering row
// added, leaving row subtracted), so both kernels give the same flow for
// the same rows per workgroup.
template <int COLS, int kM>
__global__ __launch_bounds__(COLS) void update_flow_ring_kernel(const float* __restrict__ M, int w,
                                                                int h, int ncols, int rows,
                                                                double scale,
                                                                float2* __restrict__ flow) {
    constexpr int kW = 2 * kM + 1;  // window rows = ring period
    constexpr int kRB = 5;          // rows parked in LDS per horizontal pass
    static_assert(kW % kRB == 0, "the LDS batch must divide the ring period");
    __shared__ float buf[kRB][5][COLS];
    const int tw = ncols - 2 * kM;
    const int X0 = blockIdx.x * tw;
    const int Y0 = blockIdx.y * rows;
    const int p = blockIdx.z;
    const long P = (long)w * h;
    const float* Mp = M + (long)p * 5 * P;
    float2* Fp = flow + (long)p * P;
    const int tid = threadIdx.x;
    const bool col_ok = tid < ncols;
    const int xc = min(max(X0 - kM + tid, 0), w - 1);
    // ring slot j holds the column's values of the row that entered the
    // window j rows (mod kW) after the workgroup's first window row
    float ring[5][kW];
    double vs[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int j = 0; j < kW; ++j) {
        const float* q = Mp + (long)min(max(Y0 - kM + j, 0), h - 1) * w + xc;
#pragma unroll
        for (int c = 0; c < 5; ++c) {
            ring[c][j] = col_ok ? q[c * P] : 0.f;
            vs[c] += ring[c][j];
        }
    }
    const int yend = min(Y0 + rows, h);
    const int xend = min(tw, w - X0);  // output columns of this strip
    const int runs = (xend + kBfRun - 1) / kBfRun;
    // values of the rows entering after output rows yb .. yb+kRB-1 (row
    // y+kM+1 after row y), loaded one batch ahead: their loads stay in flight
    // across the batch's horizontal pass (the barriers below wait for LDS
    // only)
    float ent[kRB][5];
    auto load_entering = [&](int yb) {
#pragma unroll
        for (int r = 0; r < kRB; ++r) {
            const int y = yb + r;
            const float* qa = Mp + (long)min(y + kM + 1, h - 1) * w + xc;
            const bool ok = col_ok && y + 1 < yend;
#pragma unroll
            for (int c = 0; c < 5; ++c) ent[r][c] = ok ? qa[c * P] : 0.f;
        }
    };
    load_entering(Y0);
    for (int yc = Y0; yc < yend; yc += kW) {
#pragma unroll
        for (int b = 0; b < kW / kRB; ++b) {
            const int yb = yc + b * kRB;
            if (yb >= yend) break;
            const int nr = min(kRB, yend - yb);
#pragma unroll
            for (int r = 0; r < kRB; ++r) {
                if (r < nr) {
#pragma unroll
                    for (int c = 0; c < 5; ++c) buf[r][c][tid] = (float)vs[c];
                    if (yb + r + 1 < yend) {
                        // row yb+r+kM+1 enters, row yb+r-kM (ring slot b*kRB + r) leaves
#pragma unroll
                        for (int c = 0; c < 5; ++c) {
                            vs[c] += (double)ent[r][c] - (double)ring[c][b * kRB + r];
                            ring[c][b * kRB + r] = ent[r][c];
                        }
                    }
                }
            }
            load_entering(yb + kRB);
            // LDS-only barrier: the entering rows' loads stay in flight
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            for (int j = tid; j < nr * runs; j += COLS) {
                const int r = j / runs;
                const int x0 = (j - r * runs) * kBfRun;
                const int n = min(kBfRun, xend - x0);
                float s[5][kBfRun];
#pragma unroll
                for (int c = 0; c < 5; ++c) {
                    const float* v = &buf[r][c][x0];
                    float a = 0.f;
#pragma unroll
                    for (int k = 0; k < kW; ++k) a += v[k];
                    s[c][0] = a;
#pragma unroll
                    for (int i = 1; i < kBfRun; ++i) {
                        if (i < n) a += v[i + 2 * kM] - v[i - 1];
                        s[c][i] = a;
                    }
                }
                float2* out = Fp + (long)(yb + r) * w + X0 + x0;
#pragma unroll
                for (int i = 0; i < kBfRun; ++i) {
                    if (i < n) {
                        const double g11 = s[0][i] * scale, g12 = s[1][i] * scale;
                        const double g22 = s[2][i] * scale, h1 = s[3][i] * scale;
                        const double h2 = s[4][i] * scale;
                        const double idet = 1.0 / (g11 * g22 - g12 * g12 + 1e-3);
                        out[i] = make_float2((float)((g11 * h2 - g12 * h1) * idet),
                                             (float)((g22 * h1 - g12 * h2) * idet));
                    }
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
    }
}

__global__ __launch_bounds__(256) void flow_cells_kernel(const float2* __restrict__ flow, int W,
                                                         int H, int rows, int cols,
                                                         float* __restrict__ cells) {
    __shared__ float colsum[kMaxSide];
    const int r = blockIdx.x, p = blockIdx.y;
    const int ch = H / rows, cw = W / cols;
    const float2* F = flow + (long)p * W * H + (long)r * ch * W;
    if ((W & 1) == 0 && (((uintptr_t)F) & 15) == 0) {
        const float4* F4 = reinterpret_cast<const float4*>(F);   // 2 pixels per load
        const int W2 = W / 2;
        for (int x2 = threadIdx.x; x2 < W2; x2 += 256) {
            float s0 = 0.f, s1 = 0.f;
#pragma unroll 4
            for (int yy = 0; yy < ch; ++yy) {
                const float4 d = F4[(long)yy * W2 + x2];
                s0 += sqrtf(d.x * d.x + d.y * d.y);
                s1 += sqrtf(d.z * d.z + d.w * d.w);
            }
            colsum[2 * x2] = s0;
            colsum[2 * x2 + 1] = s1;
        }
    } else {
        for (int x = threadIdx.x; x < W; x += 256) {
            float s = 0.f;
            for (int yy = 0; yy < ch; ++yy) {
                const float2 d = F[(long)yy * W + x];
                s += sqrtf(d.x * d.x + d.y * d.y);
            }
            colsum[x] = s;
        }
    }
    __syncthreads();
    for (int c = threadIdx.x; c < cols; c += 256) {
        float s = 0.f;
        for (int k = 0; k < cw; ++k) s += colsum[c * cw + k];
        cells[((long)p * rows + r) * cols + c] = s / (float)(ch * cw);
    }
}

__global__ __launch_bounds__(256) void tile_change_kernel(const float* __restrict__ cells,
                                                          int pairs, int tokens, int tile_tokens,
                                                          int tiles, double* __restrict__ change) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)pairs * tiles) return;
    const int p = (int)(i / tiles), t = (int)(i - (long)p * tiles);
    const int b = t * tile_tokens, e = min(b + tile_tokens, tokens);
    double s = 0.0;
    for (int k = b; k < e; ++k) s += (double)cells[(long)p * tokens + k];
    change[i] = s / (double)(e - b);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int launch_ok(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return 1;
    }
    return 0;
}

int round_half_even(double v) { return (int)std::nearbyint(v); }

struct Level {
    int k;
    double scale, sigma;
    int ksize, w, h;
};

// Levels from the coarsest to the full size (OpenCV: stop at the first
// scale where a side falls under 32 pixels).
std::vector<Level> level_plan(int W, int H, double pyr_scale, int levels) {
    double scale = 1.0;
    int k = 0;
    while (k < levels) {
        scale *= pyr_scale;
        if (W * scale < kMinLevelSide || H * scale < kMinLevelSide) break;
        ++k;
    }
    std::vector<Level> plan;
    for (int lv = k; lv >= 0; --lv) {
        double s = 1.0;
        for (int i = 0; i < lv; ++i) s *= pyr_scale;
        const double sigma = (1.0 / s - 1.0) * 0.5;
        int ksize = round_half_even(sigma * 5) | 1;
        if (ksize < 3) ksize = 3;
        plan.push_back({lv, s, sigma, ksize, round_half_even(W * s), round_half_even(H * s)});
    }
    return plan;
}

// getGaussianKernel(ksize, sigma) for fp32 images: the fixed binomial-like
// tables for ksize <= 7 and sigma <= 0, else normalised exp(-x^2 / 2 sigma^2).
bool blur_taps(int ksize, double sigma, BlurTaps& t) {
    if (ksize > kMaxBlurTaps) return false;
    t.ksize = ksize;
    static const float small[4][7] = {
        {1.f},
        {0.25f, 0.5f, 0.25f},
        {0.0625f, 0.25f, 0.375f, 0.25f, 0.0625f},
        {0.03125f, 0.109375f, 0.21875f, 0.28125f, 0.21875f, 0.109375f, 0.03125f}};
    if (sigma <= 0 && (ksize & 1) && ksize <= 7) {
        for (int i = 0; i < ksize; ++i) t.k[i] = small[ksize >> 1][i];
        return true;
    }
    if (sigma <= 0) sigma = ((ksize - 1) * 0.5 - 1) * 0.3 + 0.8;
    std::vector<double> v(ksize);
    double sum = 0;
    for (int i = 0; i < ksize; ++i) {
        const double x = i - (ksize - 1) * 0.5;
        v[i] = std::exp(-x * x / (2 * sigma * sigma));
        sum += v[i];
    }
    for (int i = 0; i < ksize; ++i) t.k[i] = (float)(v[i] / sum);
    return true;
}

// 6x6 Gauss-Jordan inverse with partial pivoting (the Gram matrix is SPD).
bool invert6(double a[6][6], double inv[6][6]) {
    for (int i = 0; i < 6; ++i)
        for (int j = 0; j < 6; ++j) inv[i][j] = i == j;
    for (int c = 0; c < 6; ++c) {
        int piv = c;
        for (int r = c + 1; r < 6; ++r)
            if (std::fabs(a[r][c]) > std::fabs(a[piv][c])) piv = r;
        if (a[piv][c] == 0) return false;
        for (int j = 0; j < 6; ++j) {
            std::swap(a[c][j], a[piv][j]);
            std::swap(inv[c][j], inv[piv][j]);
        }
        const double d = a[c][c];
        for (int j = 0; j < 6; ++j) {
            a[c][j] /= d;
            inv[c][j] /= d;
        }
        for (int r = 0; r < 6; ++r) {
            if (r == c) continue;
            const double f = a[r][c];
            for (int j = 0; j < 6; ++j) {
                a[r][j] -= f * a[c][j];
                inv[r][j] -= f * inv[c][j];
            }
        }
    }
    return true;
}

// Applicability taps and the inverse-Gram entries of the basis
// [1, x, y, x^2, y^2, xy] (FarnebackPrepareGaussian).
bool poly_taps(int n, double sigma, PolyTaps& t) {
    if (sigma < FLT_EPSILON) sigma = n * 0.3;
    t.n = n;
    double s = 0;
    for (int k = -n; k <= n; ++k) {
        t.g[k + n] = (float)std::exp(-k * k / (2 * sigma * sigma));
        s += t.g[k + n];
    }
    for (int k = -n; k <= n; ++k) {
        t.g[k + n] = (float)(t.g[k + n] / s);
        t.xg[k + n] = (float)(k * (double)t.g[k + n]);
        t.xxg[k + n] = (float)(k * k * (double)t.g[k + n]);
    }
    double G[6][6] = {};
    for (int y = -n; y <= n; ++y)
        for (int x = -n; x <= n; ++x) {
            const double gg = (double)t.g[y + n] * t.g[x + n];
            const double b[6] = {1.0, (double)x, (double)y, (double)x * x, (double)y * y,
                                 (double)x * y};
            for (int i = 0; i < 6; ++i)
                for (int j = 0; j < 6; ++j) G[i][j] += gg * b[i] * b[j];
        }
    double iG[6][6];
    if (!invert6(G, iG)) return false;
    t.ig11 = iG[1][1];
    t.ig03 = iG[0][3];
    t.ig33 = iG[3][3];
    t.ig55 = iG[5][5];
    return true;
}

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

struct Layout {
    size_t hbuf, img, R, M, fa, fb, total;
};

Layout layout(int nf, int W, int H, const std::vector<Level>& plan) {
    const size_t P0 = (size_t)W * H;
    size_t P1 = 0, hcols = W;   // row-blur output: W columns, or 2 per level column
    for (const Level& l : plan)
        if (l.k > 0) {
            P1 = std::max(P1, (size_t)l.w * l.h);
            hcols = std::max(hcols, (size_t)2 * l.w);
        }
    const size_t pairs = nf - 1;
    Layout L;
    size_t off = 0;
    L.hbuf = off; off += align256(nf * (size_t)H * hcols * sizeof(float));
    L.img = off;  off += align256(nf * P0 * sizeof(float));
    L.R = off;    off += align256(nf * 5 * P0 * sizeof(float));
    L.M = off;    off += align256(pairs * 5 * P0 * sizeof(float));
    L.fa = off;   off += align256(pairs * P1 * 2 * sizeof(float));
    L.fb = off;   off += align256(pairs * P1 * 2 * sizeof(float));
    L.total = off;
    return L;
}

// launch kinds reported by kvp_farneback_profile
enum {
    KIND_BLUR_ROWS = 0,
    KIND_BLUR_COLS_RESIZE = 1,
    KIND_POLY_EXP = 2,
    KIND_MATRICES_INIT = 3,
    KIND_FLOW = 4,
    KIND_MATRICES = 5,
};

int check_params(int nf, int W, int H, double pyr_scale, int levels, int winsize,
                 int iterations, int poly_n, int flags) {
    if (nf < 2 || nf > kMaxFrames) {
        set_error("farneback: %d frames (2..%d)", nf, kMaxFrames);
        return 1;
    }
    if (W < kMinSide || H < kMinSide || W > kMaxSide || H > kMaxSide) {
        set_error("farneback: frame %dx%d outside %d..%d per side", W, H, kMinSide, kMaxSide);
        return 1;
    }
    if (!(pyr_scale > 0 && pyr_scale < 1)) {
        set_error("farneback: pyr_scale %g must be in (0, 1)", pyr_scale);
        return 1;
    }
    if (levels < 0 || iterations < 0) {
        set_error("farneback: levels and iterations must be >= 0");
        return 1;
    }
    if (winsize < 1 || winsize / 2 > kMaxBoxHalf) {
        set_error("farneback: winsize %d outside 1..%d", winsize, 2 * kMaxBoxHalf + 1);
        return 1;
    }
    if (poly_n < 1 || poly_n > kMaxPolyN) {
        set_error("farneback: poly_n %d outside 1..%d", poly_n, kMaxPolyN);
        return 1;
    }
    if (flags != 0) {
        set_error("farneback: flags %d not supported (only 0: zero initial flow, box window)",
                  flags);
        return 1;
    }
    return 0;
}

// Launch timeline for kvp_farneback_profile: an event after every launch.
struct Timeline {
    hipStream_t st;
    std::vector<hipEvent_t> ev;
    std::vector<int> kind, level;
    bool ok = true;
    void mark(int k, int lv) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) {
            ok = false;
            return;
        }
        if (hipEventRecord(e, st) != hipSuccess) ok = false;
        ev.push_back(e);
        kind.push_back(k);
        level.push_back(lv);
    }
    ~Timeline() {
        for (hipEvent_t e : ev) (void)hipEventDestroy(e);
    }
};

int farneback_impl(const uint8_t* frames, long frame_stride, int nf, int W, int H,
                   double pyr_scale, int levels, int winsize, int iterations, int poly_n,
                   double poly_sigma, int flags, void* workspace, long workspace_bytes,
                   float* flows, void* stream_v, Timeline* tl = nullptr) {
    if (check_params(nf, W, H, pyr_scale, levels, winsize, iterations, poly_n, flags)) return 1;
    if (!frames || !flows || !workspace) {
        set_error("farneback: null pointer");
        return 1;
    }
    const std::vector<Level> plan = level_plan(W, H, pyr_scale, levels);
    const Layout L = layout(nf, W, H, plan);
    if (workspace_bytes < 0 || (size_t)workspace_bytes < L.total) {
        set_error("farneback: workspace %ld bytes < %zu needed", workspace_bytes, L.total);
        return 1;
    }
    PolyTaps pt;
    if (!poly_taps(poly_n, poly_sigma, pt)) {
        set_error("farneback: singular applicability (poly_n %d, poly_sigma %g)", poly_n,
                  poly_sigma);
        return 1;
    }
    for (const Level& l : plan) {
        if (l.ksize > kMaxBlurTaps) {
            set_error("farneback: level %d needs a %d-tap pre-blur (max %d)", l.k, l.ksize,
                      kMaxBlurTaps);
            return 1;
        }
    }
    hipStream_t st = (hipStream_t)stream_v;
    char* ws = (char*)workspace;
    float* hbuf = (float*)(ws + L.hbuf);
    float* img = (float*)(ws + L.img);
    float* R = (float*)(ws + L.R);
    float* M = (float*)(ws + L.M);
    float2* fbuf[2] = {(float2*)(ws + L.fa), (float2*)(ws + L.fb)};
    const int pairs = nf - 1;
    const int m = winsize / 2;
    const double box_scale = 1.0 / ((double)winsize * winsize);

    auto mark = [&](int kind, int lv) {
        if (tl) tl->mark(kind, lv);
    };
    mark(-1, -1);
    const float2* prev = nullptr;
    int pw = 0, ph = 0;
    for (size_t li = 0; li < plan.size(); ++li) {
        const Level& l = plan[li];
        BlurTaps bt;
        blur_taps(l.ksize, l.sigma, bt);
        const bool same = l.w == W && l.h == H;
        const int ncols = same ? W : 2 * l.w;
        const double sxs = 1.0 / ((double)l.w / W), sys = 1.0 / ((double)l.h / H);
        blur_rows_kernel<<<dim3(H, 1, nf), 256, (W + 2 * (l.ksize / 2)) * sizeof(float), st>>>(
            frames, frame_stride, W, H, hbuf, ncols, same ? 1 : 0, sxs, bt);
        mark(KIND_BLUR_ROWS, l.k);
        blur_cols_resize_kernel<<<dim3((l.w + 63) / 64, (l.h + 3) / 4, nf), 256, 0, st>>>(
            hbuf, ncols, W, H, img, l.w, l.h, sxs, sys, same ? 1 : 0, bt);
        mark(KIND_BLUR_COLS_RESIZE, l.k);
        poly_exp_kernel<<<dim3((l.w + kPeTileW - 1) / kPeTileW, (l.h + kPeTileH - 1) / kPeTileH,
                               nf),
                          256, 0, st>>>(img, l.w, l.h, R, pt);
        mark(KIND_POLY_EXP, l.k);
        if (launch_ok("farneback pyramid")) return 1;

        float2* fl = l.k == 0 ? (float2*)flows : fbuf[li & 1];
        const long P = (long)l.w * l.h;
        const dim3 pix((unsigned)((P + 255) / 256), pairs);
        const int mode = prev ? 2 : 1;
        update_matrices_kernel<<<pix, 256, 0, st>>>(
            R, l.w, l.h, fl, M, mode, prev, pw, ph, prev ? 1.0 / ((double)l.w / pw) : 1.0,
            prev ? 1.0 / ((double)l.h / ph) : 1.0, (float)(1.0 / pyr_scale),
            iterations == 0 ? 1 : 0);
        mark(KIND_MATRICES_INIT, l.k);
        // narrow levels take 128-column strips; rows per workgroup (a multiple
        // of the LDS batch, 8..32) so that a launch has ~kBfTargetGroups groups
        const bool narrow = l.w + 2 * m <= 128 || l.w < 400;
        const int cols = narrow ? 128 : 256;
        const int strips = (l.w + cols - 2 * m - 1) / (cols - 2 * m);
        // winsize 15 (the reference's): the register-ring kernel, strips
        // trimmed to the level's width, up to kBfRingRows rows per workgroup
        // (a multiple of its LDS batch) so that a launch has ~kBfRingGroups
        const bool ring = m == kBfRingHalf;
        const int ring_cols = (l.w + strips - 1) / strips + 2 * m;
        long want = ((long)l.h * strips * pairs + kBfTargetGroups - 1) / kBfTargetGroups;
        int rows = (int)std::min<long>(32, std::max<long>(kBfBatch, want));
        rows = (rows + kBfBatch - 1) / kBfBatch * kBfBatch;
        if (ring) {
            want = ((long)l.h * strips * pairs + kBfRingGroups - 1) / kBfRingGroups;
            rows = (int)std::min<long>(kBfRingRows, std::max<long>(kBfRingMinRows, want));
            rows = (rows + 4) / 5 * 5;
        }
        const dim3 box_grid(strips, (l.h + rows - 1) / rows, pairs);
        for (int it = 0; it < iterations; ++it) {
            if (ring && narrow)
                update_flow_ring_kernel<128, kBfRingHalf><<<box_grid, 128, 0, st>>>(
                    M, l.w, l.h, ring_cols, rows, box_scale, fl);
            else if (ring)
                update_flow_ring_kernel<256, kBfRingHalf><<<box_grid, 256, 0, st>>>(
                    M, l.w, l.h, ring_cols, rows, box_scale, fl);
            else if (narrow)
                update_flow_kernel<128><<<box_grid, 128, 0, st>>>(M, l.w, l.h, m, rows, box_scale,
                                                                   fl);
            else
                update_flow_kernel<256><<<box_grid, 256, 0, st>>>(M, l.w, l.h, m, rows, box_scale,
                                                                   fl);
            mark(KIND_FLOW, l.k);
            if (it < iterations - 1) {
                update_matrices_kernel<<<pix, 256, 0, st>>>(R, l.w, l.h, fl, M, 0, nullptr, 0, 0,
                                                            1.0, 1.0, 1.f, 0);
                mark(KIND_MATRICES, l.k);
            }
        }
        if (launch_ok("farneback iterations")) return 1;
        prev = fl;
        pw = l.w;
        ph = l.h;
    }
    return 0;
}

}  // namespace
}  // namespace kvp

extern "C" {

long kvp_farneback_workspace_bytes(int num_frames, int width, int height, double pyr_scale,
                                   int levels) {
    if (num_frames < 2 || width < 1 || height < 1 || !(pyr_scale > 0 && pyr_scale < 1) ||
        levels < 0)
        return -1;
    return (long)kvp::layout(num_frames, width, height,
                             kvp::level_plan(width, height, pyr_scale, levels))
        .total;
}

int kvp_farneback_flows(const unsigned char* frames, int num_frames, int width, int height,
                        double pyr_scale, int levels, int winsize, int iterations, int poly_n,
                        double poly_sigma, int flags, void* workspace, long workspace_bytes,
                        float* flows, void* stream) {
    return kvp::farneback_impl(frames, (long)width * height, num_frames, width, height,
                               pyr_scale, levels, winsize, iterations, poly_n, poly_sigma, flags,
                               workspace, workspace_bytes, flows, stream);
}

int kvp_farneback_flow(const unsigned char* prev, const unsigned char* next, float* flow,
                       int width, int height, double pyr_scale, int levels, int winsize,
                       int iterations, int poly_n, double poly_sigma, int flags, void* workspace,
                       long workspace_bytes, void* stream) {
    if (!prev || !next) {
        kvp::set_error("farneback: null frame");
        return 1;
    }
    const long stride = (long)((intptr_t)next - (intptr_t)prev);
    return kvp::farneback_impl(prev, stride, 2, width, height, pyr_scale, levels, winsize,
                               iterations, poly_n, poly_sigma, flags, workspace, workspace_bytes,
                               flow, stream);
}

int kvp_farneback_profile(const unsigned char* frames, int num_frames, int width, int height,
                          double pyr_scale, int levels, int winsize, int iterations, int poly_n,
                          double poly_sigma, int flags, void* workspace, long workspace_bytes,
                          float* flows, float* launch_ms, int* launch_kind, int* launch_level,
                          int capacity, int* count, void* stream) {
    if (!launch_ms || !launch_kind || !launch_level || !count) {
        kvp::set_error("farneback_profile: null output array");
        return 1;
    }
    kvp::Timeline tl;
    tl.st = (hipStream_t)stream;
    const int rc = kvp::farneback_impl(frames, (long)width * height, num_frames, width, height,
                                       pyr_scale, levels, winsize, iterations, poly_n,
                                       poly_sigma, flags, workspace, workspace_bytes, flows,
                                       stream, &tl);
    if (rc) return rc;
    if (!tl.ok || tl.ev.empty()) {
        kvp::set_error("farneback_profile: event creation failed");
        return 1;
    }
    if (hipEventSynchronize(tl.ev.back()) != hipSuccess) {
        kvp::set_error("farneback_profile: event synchronize failed");
        return 1;
    }
    const int n = (int)tl.ev.size() - 1;
    *count = n;
    if (n > capacity) {
        kvp::set_error("farneback_profile: %d launches > capacity %d", n, capacity);
        return 1;
    }
    for (int i = 0; i < n; ++i) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, tl.ev[i], tl.ev[i + 1]) != hipSuccess) {
            kvp::set_error("farneback_profile: elapsed time unavailable");
            return 1;
        }
        launch_ms[i] = ms;
        launch_kind[i] = tl.kind[i + 1];
        launch_level[i] = tl.level[i + 1];
    }
    return 0;
}

int kvp_motion_change_rates(const float* flows, int pairs, int width, int height, int grid_rows,
                            int grid_cols, int tile_tokens, float* cell_maps, double* change,
                            void* stream) {
    if (!flows || !cell_maps || !change) {
        kvp::set_error("change_rates: null pointer");
        return 1;
    }
    if (pairs < 1 || grid_rows < 1 || grid_cols < 1 || tile_tokens < 1 || width > kvp::kMaxSide ||
        height > kvp::kMaxSide || pairs > 65535) {
        kvp::set_error("change_rates: bad sizes");
        return 1;
    }
    if (width % grid_cols || height % grid_rows) {
        kvp::set_error("change_rates: grid %dx%d does not divide %dx%d", grid_rows, grid_cols,
                       width, height);
        return 1;
    }
    hipStream_t st = (hipStream_t)stream;
    kvp::flow_cells_kernel<<<dim3(grid_rows, pairs), 256, 0, st>>>(
        (const float2*)flows, width, height, grid_rows, grid_cols, cell_maps);
    const int tokens = grid_rows * grid_cols;
    const int tiles = (tokens + tile_tokens - 1) / tile_tokens;
    const long n = (long)pairs * tiles;
    kvp::tile_change_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(
        cell_maps, pairs, tokens, tile_tokens, tiles, change);
    return kvp::launch_ok("change_rates");
}

}  // extern "C"

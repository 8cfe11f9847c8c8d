// Upstream K/V producer of the KV-arena path, gfx950-native: the random-init
// DiT self-attention stack whose per-layer K/V the arena persists
// (reference: src/backbone.py:8-67, src/config.py:6-27).
//
//   layer_norm_kernel   nn.LayerNorm over the hidden dim (backbone.py:28,48):
//                       one wave per token row, the row held in registers,
//                       two-pass mean and biased variance in fp32.
//   init kernels        parameter init on the device: Linear weights
//                       normal(0, 0.02), Linear biases 0 (backbone.py:51-56),
//                       LayerNorm weight 1 and bias 0 (nn.LayerNorm's own
//                       init). Normals come from SplitMix64 (Steele, Lea and
//                       Flood, OOPSLA 2014) through the Box-Muller transform;
//                       the values are this library's own, not torch's.
//   linear()            y = x W^T + b (+ y) (nn.Linear, backbone.py:13-14,44):
//                       the grouped bf16 projection kernel where it tiles the
//                       shape, else the generic fp32-matrix-core kernel
//                       (proj_gemm.hip); out_proj adds into the residual
//                       stream in the epilogue.
//   Backbone            token_embed -> blocks -> final_norm (backbone.py:58-67);
//                       a block is LN -> q,k,v projections -> intra-frame
//                       attention (this library's attention kernel, the
//                       reference's F.scaled_dot_product_attention with its
//                       default 1/sqrt(head_dim) scale) -> out_proj added to
//                       the residual stream (backbone.py:16-33).
//
// Layout: token-major [rows, D], rows = frames * tokens_per_frame, the layout
// the attention kernels and the arena consume. The reference returns k, v as
// (b, heads, t, head_dim); its element (b, h, t, d) is element
// (b*T + t, h*128 + d) here. The residual stream is fp32 in both dtypes; in
// bf16 mode the weights of the two projections, the normalised activations,
// q/k/v and the attention output are bf16 (fp32 accumulation throughout).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <tuple>
#include <vector>

#include "kvp_internal.h"
#include "kvp_producer.h"

namespace kvp {
namespace {

constexpr int kLnMaxChunks = 16;    // 4 elements per lane per chunk: D <= 4096
constexpr int kLnRowsPerBlock = 4;  // one wave per row
constexpr float kLnEps = 1e-5f;     // nn.LayerNorm default
constexpr int kHeadDim = 128;
constexpr float kInitStd = 0.02f;   // reference: src/backbone.py:54

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

struct alignas(8) Bf16x4 {
    __bf16 v[4];
};

__device__ inline void load4(const float* p, float (&v)[4]) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x;
    v[1] = t.y;
    v[2] = t.z;
    v[3] = t.w;
}

__device__ inline void load4(const __bf16* p, float (&v)[4]) {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = __uint_as_float(t.x << 16);
    v[1] = __uint_as_float(t.x & 0xffff0000u);
    v[2] = __uint_as_float(t.y << 16);
    v[3] = __uint_as_float(t.y & 0xffff0000u);
}

__device__ inline void store4(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

__device__ inline void store4(__bf16* p, const float (&v)[4]) {
    Bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.v[e] = (__bf16)v[e];  // round to nearest even
    *reinterpret_cast<Bf16x4*>(p) = o;
}

__device__ inline float wave_sum(float s) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    return s;
}

// y[r, :] = (x[r, :] - mean) * rstd * gamma + beta, statistics in fp32 over
// the D elements of the row (biased variance, as nn.LayerNorm).
// NCH chunks of 256 elements per row are held in registers (NCH * 4 per
// lane); the host picks the smallest instantiated NCH with NCH * 256 >= D.
template <typename InT, typename OutT, int NCH>
__global__ __launch_bounds__(64 * kLnRowsPerBlock) void layer_norm_kernel(
    const InT* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    OutT* __restrict__ y, long rows, int D, float eps) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kLnRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const InT* xr = x + row * (long)D;
    float v[NCH][4];
    // gamma and beta are loaded with the row, so that the only memory round
    // trip before the stores is the row's own
    float g[NCH][4], b[NCH][4];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = c * 256 + lane * 4;
        if (col < D) {
            load4(xr + col, v[c]);
            load4(gamma + col, g[c]);
            load4(beta + col, b[c]);
            s += (v[c][0] + v[c][1]) + (v[c][2] + v[c][3]);
        } else {
            v[c][0] = v[c][1] = v[c][2] = v[c][3] = 0.f;
        }
    }
    // Correctly rounded divisions: a row of equal values gets its exact mean,
    // so it normalises to beta exactly.
    const float mean = wave_sum(s) / (float)D;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        if (c * 256 + lane * 4 < D) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = v[c][e] - mean;
                ss = fmaf(d, d, ss);
            }
        }
    }
    const float rstd = rsqrtf(wave_sum(ss) / (float)D + eps);
    OutT* yr = y + row * (long)D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = c * 256 + lane * 4;
        if (col < D) {
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = fmaf((v[c][e] - mean) * rstd, g[c][e], b[c][e]);
            store4(yr + col, o);
        }
    }
}

// SplitMix64: the i-th output of the generator seeded with `seed` is
// mix(seed + (i + 1) * golden).
__host__ __device__ inline uint64_t splitmix64(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// p[i] = stdv * N(0, 1) from output i of the parameter's SplitMix64 stream:
// u1 in (0, 1] from the top 24 bits, u2 in [0, 1) from the next 24,
// z = sqrt(-2 ln u1) cos(2 pi u2) (Box-Muller).
template <typename T>
__global__ void init_normal_kernel(T* __restrict__ p, long n, uint64_t key, float stdv) {
    const long step = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
        const uint64_t h = splitmix64(key, (uint64_t)i);
        const float u1 = (float)((h >> 40) + 1) * 0x1p-24f;
        const float u2 = (float)((h >> 16) & 0xffffffull) * 0x1p-24f;
        const float z = sqrtf(-2.f * logf(u1)) * cospif(2.f * u2);
        p[i] = (T)(stdv * z);
    }
}

template <typename T>
__global__ void fill_kernel(T* __restrict__ p, long n, float value) {
    const long step = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) p[i] = (T)value;
}

unsigned grid_for(long n) {
    long g = (n + 255) / 256;
    if (g > 4096) g = 4096;
    return (unsigned)(g < 1 ? 1 : g);
}

size_t dtype_size(int dt) { return dt == 1 ? 2 : 4; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int launch_ok(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s launch: %s", what, hipGetErrorString(e));
        return 1;
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Linear layers: the grouped bf16 projection kernel for the shapes it tiles
// (K % 64, N % 128, 16-byte aligned operands: every projection of the
// reference's configuration), the generic fp32-matrix-core kernel for every
// other shape and for fp32 (proj_gemm.hip). No library GEMM.
// ---------------------------------------------------------------------------

int linear_impl(int in_t, int out_t, const void* x, const void* w, const float* bias, void* y,
                long rows, int K, int N, bool acc, void* stream) {
    if (in_t == 1 && K % 64 == 0 && N % 128 == 0 && aligned16(x) && aligned16(w) &&
        aligned16(bias) && aligned16(y) && rows > 0 && (out_t == 0 || !acc)) {
        void* outs[3] = {y, nullptr, nullptr};
        const int rc = launch_proj_gemm(x, w, bias, outs, 1, rows, K, N, out_t, acc, 128, stream);
        if (rc != 2) return rc;
        clear_error();
    }
    return launch_gemm_generic(in_t, out_t, x, w, bias, y, rows, K, N, acc, stream);
}

int layer_norm_impl(int in_t, int out_t, const void* x, const float* gamma, const float* beta,
                    void* y, long rows, int D, float eps, void* stream) {
    if ((in_t != 0 && in_t != 1) || (out_t != 0 && out_t != 1)) {
        set_error("layer_norm: dtype %d -> %d not supported (0 = fp32, 1 = bf16)", in_t, out_t);
        return 1;
    }
    if (rows <= 0 || D <= 0 || D % 4 || D > kLnMaxChunks * 256) {
        set_error("layer_norm: rows=%ld D=%d (D must be a multiple of 4, at most %d)", rows, D,
                  kLnMaxChunks * 256);
        return 1;
    }
    if (!x || !gamma || !beta || !y) {
        set_error("layer_norm: null pointer");
        return 1;
    }
    if (!aligned16(x) || !aligned16(gamma) || !aligned16(beta) || !aligned16(y)) {
        set_error("layer_norm: x/gamma/beta/y must be 16-byte aligned");
        return 1;
    }
    if (!(eps >= 0.f)) {
        set_error("layer_norm: eps must be >= 0");
        return 1;
    }
    const long blocks = (rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock;
    if (blocks > 0x7fffffffL) {
        set_error("layer_norm: too many rows");
        return 1;
    }
    const dim3 grid((unsigned)blocks), block(64 * kLnRowsPerBlock);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int nch = (D + 255) / 256;
    auto go = [&](auto in_tag, auto out_tag) {
        using I = decltype(in_tag);
        using O = decltype(out_tag);
        const I* xi = static_cast<const I*>(x);
        O* yo = static_cast<O*>(y);
        if (nch <= 2)
            hipLaunchKernelGGL((layer_norm_kernel<I, O, 2>), grid, block, 0, st, xi, gamma, beta,
                               yo, rows, D, eps);
        else if (nch <= 4)
            hipLaunchKernelGGL((layer_norm_kernel<I, O, 4>), grid, block, 0, st, xi, gamma, beta,
                               yo, rows, D, eps);
        else if (nch <= 6)
            hipLaunchKernelGGL((layer_norm_kernel<I, O, 6>), grid, block, 0, st, xi, gamma, beta,
                               yo, rows, D, eps);
        else if (nch <= 8)
            hipLaunchKernelGGL((layer_norm_kernel<I, O, 8>), grid, block, 0, st, xi, gamma, beta,
                               yo, rows, D, eps);
        else if (nch <= 12)
            hipLaunchKernelGGL((layer_norm_kernel<I, O, 12>), grid, block, 0, st, xi, gamma, beta,
                               yo, rows, D, eps);
        else
            hipLaunchKernelGGL((layer_norm_kernel<I, O, kLnMaxChunks>), grid, block, 0, st, xi,
                               gamma, beta, yo, rows, D, eps);
    };
    if (in_t == 0 && out_t == 0)
        go(float{}, float{});
    else if (in_t == 0)
        go(float{}, __bf16{});
    else if (out_t == 0)
        go(__bf16{}, float{});
    else
        go(__bf16{}, __bf16{});
    return launch_ok("layer_norm");
}

int qkv_project_impl(int dtype, const float* x, const float* ln_w, const float* ln_b,
                     const void* w_qkv, const float* b_qkv, void* xn, void* q, void* k, void* v,
                     long rows, int D, void* stream) {
    if (dtype != 0 && dtype != 1) {
        set_error("qkv_project: dtype %d not supported (0 = fp32, 1 = bf16)", dtype);
        return 1;
    }
    if (!w_qkv || !b_qkv || !xn || !q || !k || !v) {
        set_error("qkv_project: null pointer");
        return 1;
    }
    if (layer_norm_impl(0, dtype, x, ln_w, ln_b, xn, rows, D, kLnEps, stream)) return 1;
    if (dtype == 1) {
        // bf16: one launch of the grouped projection kernel writes q, k and v
        void* outs[3] = {q, k, v};
        const int rc = launch_proj_gemm(xn, w_qkv, b_qkv, outs, 3, rows, D, D, 1, false, 128,
                                        stream);
        if (rc != 2) return rc;  // 2: shape outside the kernel's tiling: generic kernel
        clear_error();
    }
    const size_t es = dtype_size(dtype);
    void* outs[3] = {q, k, v};
    for (int i = 0; i < 3; ++i) {
        const char* wi = static_cast<const char*>(w_qkv) + (size_t)i * D * D * es;
        if (linear_impl(dtype, dtype, xn, wi, b_qkv + (size_t)i * D, outs[i], rows, D, D, false,
                        stream))
            return 1;
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Backbone
// ---------------------------------------------------------------------------

uint16_t bf16_bits_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

class Backbone {
  public:
    struct Param {
        std::string name;
        size_t offset = 0;  // bytes into the parameter block
        long numel = 0;
        int dtype = 0;      // 0 = fp32, 1 = bf16
        int init = 0;       // 0 = normal(0, 0.02), 1 = zeros, 2 = ones
    };

    Backbone(int dtype, int layers, int T, int D, int heads, int C, uint64_t seed)
        : dtype_(dtype), layers_(layers), T_(T), D_(D), heads_(heads), C_(C), seed_(seed) {}

    ~Backbone() {
        if (params_) (void)hipFree(params_);
        for (void* p : scratch_)
            if (p) (void)hipFree(p);
    }

    int init() {
        add("token_embed.weight", (long)D_ * C_, 0, 0);
        add("token_embed.bias", D_, 0, 1);
        for (int l = 0; l < layers_; ++l) {
            const std::string b = "blocks." + std::to_string(l) + ".";
            add(b + "norm.weight", D_, 0, 2);
            add(b + "norm.bias", D_, 0, 1);
            add(b + "attn.qkv_proj.weight", 3L * D_ * D_, dtype_, 0);
            add(b + "attn.qkv_proj.bias", 3L * D_, 0, 1);
            add(b + "attn.out_proj.weight", (long)D_ * D_, dtype_, 0);
            add(b + "attn.out_proj.bias", D_, 0, 1);
        }
        add("final_norm.weight", D_, 0, 2);
        add("final_norm.bias", D_, 0, 1);
        if (hipMalloc(&params_, bytes_) != hipSuccess) {
            params_ = nullptr;
            set_error("backbone: parameter allocation of %zu bytes failed", bytes_);
            return 1;
        }
        for (size_t i = 0; i < params_list_.size(); ++i) {
            const Param& p = params_list_[i];
            void* dst = static_cast<char*>(params_) + p.offset;
            const unsigned grid = grid_for(p.numel);
            if (p.init == 0) {
                const uint64_t key = splitmix64(seed_, i);
                if (p.dtype == 1)
                    hipLaunchKernelGGL(init_normal_kernel<__bf16>, dim3(grid), dim3(256), 0, 0,
                                       static_cast<__bf16*>(dst), p.numel, key, kInitStd);
                else
                    hipLaunchKernelGGL(init_normal_kernel<float>, dim3(grid), dim3(256), 0, 0,
                                       static_cast<float*>(dst), p.numel, key, kInitStd);
            } else {
                const float val = p.init == 2 ? 1.f : 0.f;
                if (p.dtype == 1)
                    hipLaunchKernelGGL(fill_kernel<__bf16>, dim3(grid), dim3(256), 0, 0,
                                       static_cast<__bf16*>(dst), p.numel, val);
                else
                    hipLaunchKernelGGL(fill_kernel<float>, dim3(grid), dim3(256), 0, 0,
                                       static_cast<float*>(dst), p.numel, val);
            }
            if (launch_ok("backbone init")) return 1;
        }
        if (hipStreamSynchronize(0) != hipSuccess) {
            set_error("backbone: init synchronize failed");
            return 1;
        }
        return 0;
    }

    long param_count() const {
        long n = 0;
        for (const Param& p : params_list_) n += p.numel;
        return n;
    }
    int num_tensors() const { return (int)params_list_.size(); }
    const Param* at(int i) const {
        return i >= 0 && i < (int)params_list_.size() ? &params_list_[i] : nullptr;
    }
    const Param* find(const char* name) const {
        if (!name) return nullptr;
        for (const Param& p : params_list_)
            if (p.name == name) return &p;
        return nullptr;
    }
    void* ptr(const Param& p) const { return static_cast<char*>(params_) + p.offset; }
    void* ptr(const std::string& name) const { return ptr(*find(name.c_str())); }

    int set_param(const char* name, const float* host, long numel) {
        const Param* p = find(name);
        if (!p || !host || numel != p->numel) {
            set_error("backbone: set_param(%s): unknown name or numel %ld", name ? name : "(null)",
                      numel);
            return 1;
        }
        if (p->dtype == 0)
            return hipMemcpy(ptr(*p), host, numel * 4, hipMemcpyHostToDevice) == hipSuccess
                       ? 0
                       : (set_error("backbone: set_param copy failed"), 1);
        std::vector<uint16_t> bits((size_t)numel);
        for (long i = 0; i < numel; ++i) bits[(size_t)i] = bf16_bits_rne(host[i]);
        return hipMemcpy(ptr(*p), bits.data(), numel * 2, hipMemcpyHostToDevice) == hipSuccess
                   ? 0
                   : (set_error("backbone: set_param copy failed"), 1);
    }

    int get_param(const char* name, float* host, long numel) const {
        const Param* p = find(name);
        if (!p || !host || numel != p->numel) {
            set_error("backbone: get_param(%s): unknown name or numel %ld", name ? name : "(null)",
                      numel);
            return 1;
        }
        if (p->dtype == 0)
            return hipMemcpy(host, ptr(*p), numel * 4, hipMemcpyDeviceToHost) == hipSuccess
                       ? 0
                       : (set_error("backbone: get_param copy failed"), 1);
        std::vector<uint16_t> bits((size_t)numel);
        if (hipMemcpy(bits.data(), ptr(*p), numel * 2, hipMemcpyDeviceToHost) != hipSuccess) {
            set_error("backbone: get_param copy failed");
            return 1;
        }
        for (long i = 0; i < numel; ++i) {
            const uint32_t u = (uint32_t)bits[(size_t)i] << 16;
            std::memcpy(&host[i], &u, 4);
        }
        return 0;
    }

    int forward(const float* latents, int frames, float* hidden, void* q_out, void* k_out,
                void* v_out, long layer_stride, void* stream) {
        if (frames <= 0 || !latents || !k_out || !v_out) {
            set_error("backbone forward: frames=%d and non-null latents/k_out/v_out required",
                      frames);
            return 1;
        }
        const long rows = (long)frames * T_;
        const size_t es = dtype_size(dtype_);
        if (layer_stride < rows * (long)D_ || (layer_stride * (long)es) % 16) {
            set_error("backbone forward: layer_stride %ld must be >= frames*T*D = %ld and keep "
                      "16-byte alignment",
                      layer_stride, rows * (long)D_);
            return 1;
        }
        if (!aligned16(latents) || !aligned16(k_out) || !aligned16(v_out) ||
            (q_out && !aligned16(q_out)) || (hidden && !aligned16(hidden))) {
            set_error("backbone forward: buffers must be 16-byte aligned");
            return 1;
        }
        if (ensure_scratch(rows)) return 1;
        float* x = static_cast<float*>(scratch_[0]);
        void* xn = scratch_[1];
        void* ctx = scratch_[2];
        // token_embed: the frame's latents reinterpreted as [T, C] rows
        // (reference: src/backbone.py:61-62, a reshape without a permute).
        if (linear_impl(0, 0, latents, ptr("token_embed.weight"),
                        static_cast<const float*>(ptr("token_embed.bias")), x, rows, C_, D_, false,
                        stream))
            return 1;
        const size_t lbytes = (size_t)layer_stride * es;
        for (int l = 0; l < layers_; ++l) {
            const std::string b = "blocks." + std::to_string(l) + ".";
            void* q = q_out ? static_cast<char*>(q_out) + l * lbytes : scratch_[3];
            void* k = static_cast<char*>(k_out) + l * lbytes;
            void* v = static_cast<char*>(v_out) + l * lbytes;
            if (qkv_project_impl(dtype_, x, static_cast<const float*>(ptr(b + "norm.weight")),
                                 static_cast<const float*>(ptr(b + "norm.bias")),
                                 ptr(b + "attn.qkv_proj.weight"),
                                 static_cast<const float*>(ptr(b + "attn.qkv_proj.bias")), xn, q,
                                 k, v, rows, D_, stream))
                return 1;
            // Non-causal attention within each frame (reference: src/backbone.py:20).
            if (launch_attention(dtype_, q, k, v, nullptr, nullptr, ctx, T_, D_, heads_, frames,
                                 (long)T_ * D_, (long)T_ * D_, 0, 0, T_, stream))
                return 1;
            // x += ctx out_proj^T + bias (reference: src/backbone.py:22,32-33).
            if (linear_impl(dtype_, 0, ctx, ptr(b + "attn.out_proj.weight"),
                            static_cast<const float*>(ptr(b + "attn.out_proj.bias")), x, rows, D_,
                            D_, true, stream))
                return 1;
        }
        if (hidden &&
            layer_norm_impl(0, 0, x, static_cast<const float*>(ptr("final_norm.weight")),
                            static_cast<const float*>(ptr("final_norm.bias")), hidden, rows, D_,
                            kLnEps, stream))
            return 1;
        return 0;
    }

  private:
    void add(const std::string& name, long numel, int dtype, int init) {
        Param p;
        p.name = name;
        p.numel = numel;
        p.dtype = dtype;
        p.init = init;
        p.offset = bytes_;
        bytes_ += ((size_t)numel * dtype_size(dtype) + 255) & ~(size_t)255;
        params_list_.push_back(p);
    }

    // x (fp32), xn, ctx and q (model dtype), each [rows, D]; grown on demand.
    int ensure_scratch(long rows) {
        if (rows <= scratch_rows_) return 0;
        (void)hipDeviceSynchronize();
        for (void*& p : scratch_) {
            if (p) (void)hipFree(p);
            p = nullptr;
        }
        scratch_rows_ = 0;
        const size_t n = (size_t)rows * D_;
        const size_t sizes[4] = {n * 4, n * dtype_size(dtype_), n * dtype_size(dtype_),
                                 n * dtype_size(dtype_)};
        for (int i = 0; i < 4; ++i) {
            if (hipMalloc(&scratch_[i], sizes[i]) != hipSuccess) {
                scratch_[i] = nullptr;
                set_error("backbone: scratch allocation of %zu bytes failed", sizes[i]);
                return 1;
            }
        }
        scratch_rows_ = rows;
        return 0;
    }

    int dtype_, layers_, T_, D_, heads_, C_;
    uint64_t seed_;
    std::vector<Param> params_list_;
    size_t bytes_ = 0;
    void* params_ = nullptr;
    void* scratch_[4] = {nullptr, nullptr, nullptr, nullptr};
    long scratch_rows_ = 0;
};

Backbone* B(void* p) { return static_cast<Backbone*>(p); }

}  // namespace
}  // namespace kvp

extern "C" {

int kvp_layer_norm(int in_dtype, int out_dtype, const void* x, const float* gamma,
                   const float* beta, void* y, long rows, int D, float eps, void* stream) {
    return kvp::layer_norm_impl(in_dtype, out_dtype, x, gamma, beta, y, rows, D, eps, stream);
}

int kvp_linear(int in_dtype, int out_dtype, const void* x, const void* w, const float* bias,
               void* y, long rows, int in_features, int out_features, int accumulate,
               void* stream) {
    return kvp::linear_impl(in_dtype, out_dtype, x, w, bias, y, rows, in_features, out_features,
                            accumulate != 0, stream);
}

int kvp_qkv_project(int dtype, const float* x, const float* ln_weight, const float* ln_bias,
                    const void* qkv_weight, const float* qkv_bias, void* xn, void* q, void* k,
                    void* v, long rows, int D, void* stream) {
    return kvp::qkv_project_impl(dtype, x, ln_weight, ln_bias, qkv_weight, qkv_bias, xn, q, k, v,
                                 rows, D, stream);
}

void* kvp_backbone_create(int dtype, int num_layers, int tokens_per_frame, int hidden_dim,
                          int num_heads, int latent_channels, unsigned long seed) {
    if ((dtype != 0 && dtype != 1) || num_layers <= 0 || tokens_per_frame <= 0 ||
        num_heads <= 0 || latent_channels <= 0 || hidden_dim != num_heads * kvp::kHeadDim ||
        hidden_dim > kvp::kLnMaxChunks * 256) {
        kvp::set_error("backbone: bad config (dtype=%d layers=%d T=%d hidden=%d heads=%d "
                       "channels=%d; hidden must be heads * 128 and at most %d)",
                       dtype, num_layers, tokens_per_frame, hidden_dim, num_heads,
                       latent_channels, kvp::kLnMaxChunks * 256);
        return nullptr;
    }
    auto* b = new (std::nothrow) kvp::Backbone(dtype, num_layers, tokens_per_frame, hidden_dim,
                                               num_heads, latent_channels, (uint64_t)seed);
    if (!b) return nullptr;
    if (b->init()) {
        delete b;
        return nullptr;
    }
    return b;
}

void kvp_backbone_destroy(void* bb) { delete kvp::B(bb); }

long kvp_backbone_param_count(void* bb) { return bb ? kvp::B(bb)->param_count() : -1; }

int kvp_backbone_num_tensors(void* bb) { return bb ? kvp::B(bb)->num_tensors() : -1; }

const char* kvp_backbone_tensor_name(void* bb, int index) {
    const kvp::Backbone::Param* p = bb ? kvp::B(bb)->at(index) : nullptr;
    return p ? p->name.c_str() : nullptr;
}

int kvp_backbone_param_info(void* bb, const char* name, void** dev_ptr, long* numel,
                            int* dtype) {
    const kvp::Backbone::Param* p = bb ? kvp::B(bb)->find(name) : nullptr;
    if (!p) {
        kvp::set_error("backbone: unknown parameter %s", name ? name : "(null)");
        return 1;
    }
    if (dev_ptr) *dev_ptr = kvp::B(bb)->ptr(*p);
    if (numel) *numel = p->numel;
    if (dtype) *dtype = p->dtype;
    return 0;
}

int kvp_backbone_set_param(void* bb, const char* name, const float* host, long numel) {
    return bb ? kvp::B(bb)->set_param(name, host, numel) : 1;
}

int kvp_backbone_get_param(void* bb, const char* name, float* host, long numel) {
    return bb ? kvp::B(bb)->get_param(name, host, numel) : 1;
}

int kvp_backbone_forward(void* bb, const float* latents, int frames, float* hidden, void* q_out,
                         void* k_out, void* v_out, long layer_stride, void* stream) {
    if (!bb) {
        kvp::set_error("backbone forward: null backbone");
        return 1;
    }
    return kvp::B(bb)->forward(latents, frames, hidden, q_out, k_out, v_out, layer_stride,
                               stream);
}

}  // extern "C"

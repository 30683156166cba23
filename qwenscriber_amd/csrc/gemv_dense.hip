// f16 and f32 weights: the Matrix.apply .f16 / .f32 arms (kernels.zig:160-206,
// linearF16 :82-112, linearF32 :54-80). out[t][r] = sum_k w[r][k] x[t][k],
// each f16 weight widened exactly to f32 (half_float.zig:20-23 fromF16), f32
// products and sums (the reference sums in dotF32's four-lane order,
// kernels.zig:38-51; this sum runs over a wavefront's lanes, within f32
// rounding of it).
//
// HBM bound: the weights stream once per group of up to four tokens (two for
// rows of more than 4092 values, one beyond 8188). Each
// workgroup forms its tokens' activations in LDS once (as they are, or after
// RMSNorm, math.zig:118-130), and its wavefronts walk rows grid-stride: lane
// l takes the row's 16-byte slices l, l + 64, ... (8 f16 or 4 f32 values),
// four slices' loads in flight at a time, multiplies each slice by every
// token's activations and the row sums are reduced over the wavefront. For
// f16 rows the activations of a slice's two 16-byte halves sit in two LDS
// planes so that the lanes' LDS reads are consecutive 16-byte words. Rows
// that are not whole 16-byte slices, or a plane that is not 16-byte aligned,
// take the element-wise form. Epilogues as the q4 GEMV: + residual, or
// siluMul of gate / up row pairs (kernels.zig:233-239).
#include "common.h"
#include "device.h"

namespace qwh {
namespace {

struct DenseArgs {
    const uint8_t *w;       // rows x cols f16 or f32, row major
    uint32_t rows, cols;
    uint32_t tokens;
    const float *x;         // tokens x cols
    const float *norm;      // RmsNorm form: cols weights
    float eps;
    float *out;             // tokens x rows (pairs: tokens x rows / 2)
    const float *residual;  // optional, tokens x rows (not with pairs); may alias out
    uint32_t pairs;
};

// The widest rows a workgroup of TOK tokens takes: its activations and
// partial sums fill at most 64 KiB of LDS.
constexpr uint32_t dense_max_cols(int tok) { return (65536u - 16u * (uint32_t)tok) / (4u * (uint32_t)tok); }

template <bool Half>
__device__ __forceinline__ float dense_weight(const uint8_t *w, size_t i) {
    if constexpr (Half) return dev::f16_bits_to_f32(reinterpret_cast<const uint16_t *>(w)[i]);
    else return reinterpret_cast<const float *>(w)[i];
}

// Sum of one 16-byte slice's products with its activations: lo holds the
// first four (f16: values 0-3 of the slice, f32: all four), hi values 4-7.
template <bool Half>
__device__ __forceinline__ float slice_dot(const uint4 v, const float4 lo, const float4 hi) {
    float s;
    if constexpr (Half) {
        s = dev::f16_bits_to_f32((uint16_t)(v.x & 0xffffu)) * lo.x;
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.x >> 16)), lo.y, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.y & 0xffffu)), lo.z, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.y >> 16)), lo.w, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.z & 0xffffu)), hi.x, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.z >> 16)), hi.y, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.w & 0xffffu)), hi.z, s);
        s = fmaf(dev::f16_bits_to_f32((uint16_t)(v.w >> 16)), hi.w, s);
    } else {
        (void)hi;
        s = __uint_as_float(v.x) * lo.x;
        s = fmaf(__uint_as_float(v.y), lo.y, s);
        s = fmaf(__uint_as_float(v.z), lo.z, s);
        s = fmaf(__uint_as_float(v.w), lo.w, s);
    }
    return s;
}

// Row `row` times each of the TOK tokens' activations in LDS (token t's at
// xs + t * cols, in the sliced layout when `sliced`), complete in every lane.
template <bool Half, int TOK>
__device__ __forceinline__ void row_dot(const DenseArgs &a, const float *xs, uint32_t row, bool sliced, int lane,
                                        float (&s)[TOK]) {
    constexpr uint32_t kPer = Half ? 8 : 4;  // values per 16-byte slice
    const size_t elem = Half ? 2 : 4;
    const uint8_t *base = a.w + (size_t)row * a.cols * elem;
#pragma unroll
    for (int t = 0; t < TOK; ++t) s[t] = 0.0f;
    if (sliced) {
        const uint32_t slices = a.cols / kPer;
        const uint32_t hi_off = Half ? a.cols / 2 : 0;
        const uint4 *src = reinterpret_cast<const uint4 *>(base);
        for (uint32_t c0 = lane; c0 < slices; c0 += 4 * 64) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                // Slices past the row load its last slice again (not used).
                const uint32_t c = min(c0 + 64u * u, slices - 1);
                v[u] = src[c];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t c = c0 + 64u * u;
                if (c < slices) {
#pragma unroll
                    for (int t = 0; t < TOK; ++t) {
                        const float *xt = xs + (size_t)t * a.cols + c * 4;
                        const float4 lo = *reinterpret_cast<const float4 *>(xt);
                        const float4 hi = Half ? *reinterpret_cast<const float4 *>(xt + hi_off) : lo;
                        s[t] += slice_dot<Half>(v[u], lo, hi);
                    }
                }
            }
        }
    } else {
        for (uint32_t k = lane; k < a.cols; k += 64) {
            const float w = dense_weight<Half>(base, k);
#pragma unroll
            for (int t = 0; t < TOK; ++t) s[t] = fmaf(w, xs[(size_t)t * a.cols + k], s[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TOK; ++t) s[t] = dev::wave_sum(s[t]);
}

// s[lane] for lanes below TOK (a register select, no indexed access).
template <int TOK>
__device__ __forceinline__ float lane_pick(const float (&s)[TOK], int lane) {
    float y = s[0];
#pragma unroll
    for (int t = 1; t < TOK; ++t)
        if (lane == t) y = s[t];
    return y;
}

template <bool Half, bool Norm, int TOK>
__global__ __launch_bounds__(256) void gemv_dense_kernel(const DenseArgs a) {
    extern __shared__ float4 lds4[];
    float *xs = reinterpret_cast<float *>(lds4);  // TOK x cols activations, then TOK x 4 partial sums
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t cols = a.cols;
    const uint32_t first = blockIdx.y * TOK;
    constexpr uint32_t kPer = Half ? 8 : 4;
    const bool sliced = cols % kPer == 0 && ((uintptr_t)a.w & 15u) == 0;
    // Token groups past the last token repeat it (their sums are not stored).
    uint32_t token[TOK];
#pragma unroll
    for (int t = 0; t < TOK; ++t) token[t] = min(first + t, a.tokens - 1);
    float inv[TOK];
    if constexpr (Norm) {
        // math.zig:118-130: x * (1 / sqrt(mean(x^2) + eps)) * w, the sum of
        // squares reduced over the block (threads, then the four waves in
        // order).
        float *partial = xs + (size_t)TOK * cols;
#pragma unroll
        for (int t = 0; t < TOK; ++t) {
            const float *x = a.x + (size_t)token[t] * cols;
            float ss = 0.0f;
            for (uint32_t k = tid; k < cols; k += 256) ss = __fadd_rn(ss, __fmul_rn(x[k], x[k]));
            ss = dev::wave_sum(ss);
            if (lane == 0) partial[t * 4 + (tid >> 6)] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < TOK; ++t) {
            const float *p = partial + t * 4;
            const float ss = ((p[0] + p[1]) + p[2]) + p[3];
            inv[t] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)cols), a.eps)));
        }
    }
    // f16 slices: value j of slice c at c * 4 + (j & 3), in the second plane
    // (cols / 2 further on) for j >= 4.
    const bool split = Half && sliced;
#pragma unroll
    for (int t = 0; t < TOK; ++t) {
        const float *x = a.x + (size_t)token[t] * cols;
        float *dst = xs + (size_t)t * cols;
        for (uint32_t k = tid; k < cols; k += 256) {
            float v = x[k];
            if constexpr (Norm) v = __fmul_rn(__fmul_rn(v, inv[t]), a.norm[k]);
            const uint32_t idx = split ? ((k & 4u) ? cols / 2 : 0u) + (k >> 3) * 4 + (k & 3u) : k;
            dst[idx] = v;
        }
    }
    __syncthreads();
    const uint32_t wave = blockIdx.x * 4 + (tid >> 6), nwaves = gridDim.x * 4;
    const uint32_t outputs = a.pairs ? a.rows / 2 : a.rows;
    const bool store = lane < TOK && first + lane < a.tokens;
    const uint32_t my_token = first + (uint32_t)lane;
    for (uint32_t o = wave; o < outputs; o += nwaves) {
        if (a.pairs) {
            float g[TOK], u[TOK];
            row_dot<Half, TOK>(a, xs, 2 * o, sliced, lane, g);
            row_dot<Half, TOK>(a, xs, 2 * o + 1, sliced, lane, u);
            const float gv = lane_pick<TOK>(g, lane), uv = lane_pick<TOK>(u, lane);
            if (store) a.out[(size_t)my_token * outputs + o] = __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv))), uv);
        } else {
            float y[TOK];
            row_dot<Half, TOK>(a, xs, o, sliced, lane, y);
            const float yv = lane_pick<TOK>(y, lane);
            if (store) {
                const size_t at = (size_t)my_token * a.rows + o;
                a.out[at] = a.residual ? a.residual[at] + yv : yv;
            }
        }
    }
}

template <int TOK>
void launch_dense(hipStream_t s, dim3 grid, size_t lds, bool half, bool norm, const DenseArgs &a) {
    if (half && norm) gemv_dense_kernel<true, true, TOK><<<grid, 256, lds, s>>>(a);
    else if (half) gemv_dense_kernel<true, false, TOK><<<grid, 256, lds, s>>>(a);
    else if (norm) gemv_dense_kernel<false, true, TOK><<<grid, 256, lds, s>>>(a);
    else gemv_dense_kernel<false, false, TOK><<<grid, 256, lds, s>>>(a);
}

// f16 bits of each value, round to nearest even (half_float.zig:12-16).
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float *in, uint64_t count, uint16_t *out) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (uint64_t)gridDim.x * 256)
        out[i] = dev::f32_to_f16_bits(in[i]);
}

}  // namespace

bool gemv_dense_supported(int format, uint32_t cols) {
    return is_dense_format(format) && cols >= 1 && cols <= kDenseMaxCols;
}

hipError_t launch_gemv_dense(hipStream_t s, int cus, const GemvInput &in, const Matrix &w, uint32_t tokens,
                             float *out, const float *residual) {
    if (!gemv_dense_supported(w.format, w.cols) || tokens == 0) return hipErrorInvalidValue;
    if (in.mode != GemvInput::F32 && in.mode != GemvInput::RmsNorm) return hipErrorNotSupported;
    if ((in.pairs && ((w.rows & 1u) || residual)) || !in.x || !out || (in.mode == GemvInput::RmsNorm && !in.norm))
        return hipErrorInvalidValue;
    if (w.rows == 0) return hipSuccess;
    DenseArgs a{};
    a.w = w.data;
    a.rows = w.rows;
    a.cols = w.cols;
    a.tokens = tokens;
    a.x = in.x;
    a.norm = in.norm;
    a.eps = in.eps;
    a.out = out;
    a.residual = residual;
    a.pairs = in.pairs ? 1u : 0u;
    // Tokens per workgroup: four, or two for rows too wide for four (one
    // pass over the weights per group), or one.
    const int tok = tokens >= 2 && w.cols <= dense_max_cols(4) ? 4 : tokens >= 2 && w.cols <= dense_max_cols(2) ? 2 : 1;
    const uint32_t groups = (tokens + tok - 1) / tok;
    if (groups > 65535) return hipErrorInvalidValue;
    // About eight workgroups per CU in all: with many token groups each
    // workgroup walks more rows (its activations staged once for them).
    const uint32_t outputs = in.pairs ? w.rows / 2 : w.rows;
    const uint32_t target = (uint32_t)(cus > 0 ? cus : 256) * 8;
    uint32_t blocks = (target + groups - 1) / groups;
    const uint32_t most = (outputs + 3) / 4;
    if (blocks > most) blocks = most;
    if (blocks == 0) blocks = 1;
    const dim3 grid(blocks, groups);
    const size_t lds = (size_t)tok * ((size_t)w.cols + 4) * sizeof(float);
    const bool half = w.format == QWH_FORMAT_F16;
    const bool norm = in.mode == GemvInput::RmsNorm;
    if (tok == 4) launch_dense<4>(s, grid, lds, half, norm, a);
    else if (tok == 2) launch_dense<2>(s, grid, lds, half, norm, a);
    else launch_dense<1>(s, grid, lds, half, norm, a);
    return hipGetLastError();
}

hipError_t launch_f32_to_f16(hipStream_t s, const float *in, uint64_t count, uint16_t *out) {
    if (count == 0) return hipSuccess;
    uint64_t blocks = (count + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    f32_to_f16_kernel<<<(uint32_t)blocks, 256, 0, s>>>(in, count, out);
    return hipGetLastError();
}

}  // namespace qwh

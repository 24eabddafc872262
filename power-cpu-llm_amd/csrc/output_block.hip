// The attention output block on gfx950: projected = W_o . attended, then
// result = residual + rms_norm(projected, post_scale) (src/engine/
// attention.rs:866-884; project_streamed / project_streamed_batch_with over
// p9_ref_matvec, src/kernels/portable/reference.rs:36-78).
//
// The engine's exact projection sums f64 products of f32 weights and inputs
// (each product is exact in f64) per output row. Both projection kernels here
// accumulate in f64 as well, in their own order, so a projected value is the
// f32 rounding of nearly the same f64 sum: it equals the engine's except when
// the two f64 sums straddle an f32 rounding boundary, and a sum like
// 2^24 + 1 - 2^24 stays exact.
//
//   project_rows_kernel: few tokens (decode, verification). HBM-bound on the
//     weights: one wave per output row streams the row once with 16-byte
//     loads, 4096 columns in flight at a time, and keeps one f64 accumulator
//     per token per lane; the tokens' inputs come from L2.
//   project_row_lds_kernel: one token (decode), input rows up to 16384
//     wide: as project_rows_kernel<1>, with the input row staged once per
//     workgroup in LDS (requested ahead of the weights) instead of read from
//     L2 by every wave.
//   project_tiles_kernel: many tokens (prompt). MFMA-bound: 128 x 128 output
//     tiles, 32-column K steps double-buffered in LDS as f32, the products on
//     v_mfma_f64_16x16x4f64 after converting the operands to f64.
//   post_norm_kernel: one workgroup per token: the row's f64 sum of squares
//     (per-thread partial sums, then a fixed tree of lane shuffles and the
//     four waves), inv = 1/sqrt(ms + eps) in f64, y = f32(x * inv) * scale,
//     result = residual + y (f32).
#include "attention_device.hpp"
#include "context.hpp"
#include "pcl_attention.h"

#include <cstdio>

namespace pcl {

constexpr int kErrBlock = 8; // non-finite value in the output block

struct BlockParams {
    const float *x;     // attended rows [n][in]
    const float *w;     // weights [out][in]
    float *proj;        // projected rows [n][out]
    const float *scale; // post-norm scale [out]
    const float *res;   // residual rows [n][out]
    float *result;      // [n][out]
    int n, in, out;
    float eps;
    int *err;
};

constexpr int kRowTokens = 16; // tokens per pass of the row kernel

// One wave per output row; tokens [t0, t0 + min(NT, n - t0)) per launch
// pass. Instantiated for NT = 1, 2, 4, 8 and 16: a one-token decode then
// carries no per-token tests for 15 absent tokens in its inner loop (that
// made the 2816 x 4096 projection 15 us against 9 us). Every token's f64 sum
// runs in the same order in every instantiation.
template <int NT>
__global__ __launch_bounds__(256) void project_rows_kernel(BlockParams p, int t0)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= p.out)
        return;
    const int nt = p.n - t0 < NT ? p.n - t0 : NT;
    const float *wr = p.w + (int64_t)r * p.in;
    double acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
        acc[t] = 0.0;
    // 16-byte steps of the row: 4096 columns (16 per lane) in flight at once,
    // so a wave's row costs one memory round trip
    const int vecs = p.in / 4;
    int v = lane;
    for (; v + 960 < vecs; v += 1024) {
        f4 wv[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
            wv[k] = ldg4_stream(wr + 4 * (v + 64 * k));
#pragma unroll
        for (int k = 0; k < 16; ++k) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t < nt) {
                    const f4 xv = ldg4(p.x + (int64_t)(t0 + t) * p.in + 4 * (v + 64 * k));
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[t] = __builtin_fma((double)wv[k][e], (double)xv[e], acc[t]);
                }
            }
        }
    }
    for (; v < vecs; v += 64) {
        const f4 wv = ldg4_stream(wr + 4 * v);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t < nt) {
                const f4 xv = ldg4(p.x + (int64_t)(t0 + t) * p.in + 4 * v);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[t] = __builtin_fma((double)wv[e], (double)xv[e], acc[t]);
            }
        }
    }
    // columns past the last whole 16-byte step
    for (int c = 4 * vecs + lane; c < p.in; c += 64) {
        const double wc = (double)ldg(wr + c);
#pragma unroll
        for (int t = 0; t < NT; ++t)
            if (t < nt)
                acc[t] = __builtin_fma(wc, (double)ldg(p.x + (int64_t)(t0 + t) * p.in + c), acc[t]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (t < nt) {
            double s = acc[t];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1)
                s += __shfl_xor(s, o);
            acc[t] = s;
        }
    }
    if (lane < nt) {
        double mine = 0.0;
#pragma unroll
        for (int t = 0; t < NT; ++t)
            mine = lane == t ? acc[t] : mine;
        stg(p.proj + (int64_t)(t0 + lane) * p.out + r, (float)mine);
    }
}

// 128 x 128 output tile per 256-thread workgroup (2 x 2 waves of 64 x 64),
// K in steps of 32 columns, LDS rows padded to 36 floats (16-byte aligned,
// and the 16 rows an MFMA operand read touches fall in distinct banks).
constexpr int kTileM = 128, kTileN = 128, kTileK = 32, kLdsRow = 36;

typedef double d4 __attribute__((ext_vector_type(4)));

// Two workgroups per CU (2 x 72 KiB of LDS; registers held to 256 per lane,
// which also keeps the f64 accumulators out of AGPRs): 16 % faster than one
// on a 4K-token projection, where the other workgroup hides a wave's LDS and
// conversion latency between MFMAs.
__global__ __launch_bounds__(256, 2) void project_tiles_kernel(BlockParams p)
{
    __shared__ __attribute__((aligned(16))) float sa[2][kTileM * kLdsRow];
    __shared__ __attribute__((aligned(16))) float sb[2][kTileN * kLdsRow];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int m0 = blockIdx.y * kTileM, n0 = blockIdx.x * kTileN;

    // global -> registers -> LDS: each thread moves 4 float4 of A and 4 of B
    // per K step; the next step's loads are in flight during this step's MFMAs
    f4 ra[4], rb[4];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + 256 * i; // row = idx / 8, quad = idx % 8
            const int row = idx >> 3, q = idx & 7;
            const int k = k0 + 4 * q;
            ra[i] = f4{0.f, 0.f, 0.f, 0.f};
            rb[i] = f4{0.f, 0.f, 0.f, 0.f};
            if (m0 + row < p.n) {
                const float *src = p.x + (int64_t)(m0 + row) * p.in;
                if (k + 3 < p.in)
                    ra[i] = ldg4(src + k);
                else
                    for (int e = 0; e < 4; ++e)
                        ra[i][e] = k + e < p.in ? ldg(src + k + e) : 0.f;
            }
            if (n0 + row < p.out) {
                const float *src = p.w + (int64_t)(n0 + row) * p.in;
                if (k + 3 < p.in)
                    rb[i] = ldg4_stream(src + k);
                else
                    for (int e = 0; e < 4; ++e)
                        rb[i][e] = k + e < p.in ? ldg(src + k + e) : 0.f;
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + 256 * i;
            const int row = idx >> 3, q = idx & 7;
            *(f4 *)(sa[buf] + row * kLdsRow + 4 * q) = ra[i];
            *(f4 *)(sb[buf] + row * kLdsRow + 4 * q) = rb[i];
        }
    };

    d4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = d4{0.0, 0.0, 0.0, 0.0};

    const int steps = (p.in + kTileK - 1) / kTileK;
    load(0);
    store(0);
    __syncthreads();
    const int r16 = lane & 15, kq = lane >> 4;
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        if (s + 1 < steps)
            load((s + 1) * kTileK);
#pragma unroll
        for (int kc = 0; kc < kTileK; kc += 16) {
            // MFMA k slot kq of step j holds column kc + 4 kq + j
            f4 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = *(const f4 *)(sa[buf] + (wm + 16 * i + r16) * kLdsRow + kc + 4 * kq);
                b[i] = *(const f4 *)(sb[buf] + (wn + 16 * i + r16) * kLdsRow + kc + 4 * kq);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj)
                        acc[i][jj] = __builtin_amdgcn_mfma_f64_16x16x4f64(
                            (double)a[i][j], (double)b[jj][j], acc[i][jj], 0, 0, 0);
        }
        if (s + 1 < steps)
            store(buf ^ 1); // read last in step s - 1, before that step's barrier
        __syncthreads();
    }
    // acc[i][jj][e]: row wm + 16i + kq + 4e, column wn + 16 jj + r16 (the f64
    // MFMA's output rows interleave by lane group, unlike the f32 one's)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = m0 + wm + 16 * i + kq + 4 * e;
            if (row >= p.n)
                continue;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int col = n0 + wn + 16 * jj + r16;
                if (col < p.out)
                    stg(p.proj + (int64_t)row * p.out + col, (float)acc[i][jj][e]);
            }
        }
}

// One 256-thread workgroup per token row; rows up to 4096 wide stay in
// registers between the sum of squares and the output.
constexpr int kNormPer = 16;

__global__ __launch_bounds__(256) void post_norm_kernel(BlockParams p)
{
    __shared__ double part[4];
    const int t = blockIdx.x;
    const int tid = threadIdx.x;
    const float *x = p.proj + (int64_t)t * p.out;
    const float *res = p.res + (int64_t)t * p.out;
    float *y = p.result + (int64_t)t * p.out;
    const bool cached = p.out <= 256 * kNormPer;
    float xv[kNormPer], rv[kNormPer], sv[kNormPer];
    double sum = 0.0;
    bool bad = false;
    if (cached) {
#pragma unroll
        for (int k = 0; k < kNormPer; ++k) {
            const int c = tid + 256 * k;
            xv[k] = c < p.out ? ldg(x + c) : 0.f;
            rv[k] = c < p.out ? ldg(res + c) : 0.f;
            sv[k] = c < p.out ? ldg(p.scale + c) : 0.f;
        }
#pragma unroll
        for (int k = 0; k < kNormPer; ++k) {
            bad |= !is_finite(xv[k]);
            sum = __builtin_fma((double)xv[k], (double)xv[k], sum);
        }
    } else {
        for (int c = tid; c < p.out; c += 256) {
            const float v = ldg(x + c);
            bad |= !is_finite(v);
            sum = __builtin_fma((double)v, (double)v, sum);
        }
    }
    // the block's sum: a fixed tree over lanes, then over the four waves
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        sum += __shfl_xor(sum, o);
    if ((tid & 63) == 0)
        part[tid >> 6] = sum;
    __syncthreads();
    const double total = (part[0] + part[1]) + (part[2] + part[3]);
    const double inv = 1.0 / __builtin_sqrt(total / (double)p.out + (double)p.eps);
    if (cached) {
#pragma unroll
        for (int k = 0; k < kNormPer; ++k) {
            const int c = tid + 256 * k;
            if (c < p.out) {
                const float r = rv[k] + (float)((double)xv[k] * inv) * sv[k];
                bad |= !is_finite(r);
                stg(y + c, r);
            }
        }
    } else {
        for (int c = tid; c < p.out; c += 256) {
            const float normed = (float)((double)ldg(x + c) * inv) * ldg(p.scale + c);
            const float r = ldg(res + c) + normed;
            bad |= !is_finite(r);
            stg(y + c, r);
        }
    }
    if (bad)
        atomicOr(p.err, kErrBlock);
}

// The largest input row project_row_lds_kernel stages (64 KiB of LDS).
constexpr int kLdsRowFloats = 16384;

// One token t0 (p.in % 4 == 0, p.in <= kLdsRowFloats), one wave per output
// row as in project_rows_kernel<1> (the same f64 sums in the same order):
// the workgroup stages the input row in LDS once, its first 4096 columns
// requested before the rows' first weights so that the LDS stores wait only
// for them.
__global__ __launch_bounds__(256) void project_row_lds_kernel(BlockParams p, int t0)
{
    extern __shared__ f4 xs[];
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int vecs = p.in / 4;
    const bool live = r < p.out;
    // a wave past the last row streams row 0 (in bounds; unused)
    const float *wr = p.w + (int64_t)(live ? r : 0) * p.in;
    const float *xr = p.x + (int64_t)t0 * p.in;
    f4 wv[16];
    int v = lane;
    if (vecs >= 1024) {
        f4 t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            t[j] = ldg4(xr + 4 * (threadIdx.x + 256 * j));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 16; ++k)
            wv[k] = ldg4_stream(wr + 4 * (v + 64 * k));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            xs[threadIdx.x + 256 * j] = t[j];
        if (vecs > 1024)
            for (int i = 1024 + threadIdx.x; i < vecs; i += 256)
                xs[i] = ldg4(xr + 4 * i);
    } else {
        for (int i = threadIdx.x; i < vecs; i += 256)
            xs[i] = ldg4(xr + 4 * i);
    }
    __syncthreads();
    if (!live)
        return;
    double acc = 0.0;
    for (; v + 960 < vecs; v += 1024) {
        // the first step's weights are in flight already when every lane
        // takes it (vecs >= 1024); below that only lanes lane + 960 < vecs
        // take it, and request them here
        if (v != lane || vecs < 1024) {
#pragma unroll
            for (int k = 0; k < 16; ++k)
                wv[k] = ldg4_stream(wr + 4 * (v + 64 * k));
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const f4 xv = xs[v + 64 * k];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                acc = __builtin_fma((double)wv[k][e], (double)xv[e], acc);
        }
    }
    for (; v < vecs; v += 64) {
        const f4 w1 = ldg4_stream(wr + 4 * v);
        const f4 xv = xs[v];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            acc = __builtin_fma((double)w1[e], (double)xv[e], acc);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        acc += __shfl_xor(acc, o);
    if (lane == 0)
        stg(p.proj + (int64_t)t0 * p.out + r, (float)acc);
}

hipError_t launch_output_block(const BlockParams &p, hipStream_t stream)
{
    if (p.n <= 2 * kRowTokens) {
        const dim3 grid((p.out + 3) / 4);
        for (int t0 = 0; t0 < p.n; t0 += kRowTokens) {
            const int nt = p.n - t0 < kRowTokens ? p.n - t0 : kRowTokens;
            if (nt == 1 && p.in % 4 == 0 && p.in <= kLdsRowFloats)
                project_row_lds_kernel<<<grid, 256, p.in * 4, stream>>>(p, t0);
            else if (nt == 1)
                project_rows_kernel<1><<<grid, 256, 0, stream>>>(p, t0);
            else if (nt == 2)
                project_rows_kernel<2><<<grid, 256, 0, stream>>>(p, t0);
            else if (nt <= 4)
                project_rows_kernel<4><<<grid, 256, 0, stream>>>(p, t0);
            else if (nt <= 8)
                project_rows_kernel<8><<<grid, 256, 0, stream>>>(p, t0);
            else
                project_rows_kernel<16><<<grid, 256, 0, stream>>>(p, t0);
        }
    } else {
        const dim3 grid((p.out + kTileN - 1) / kTileN, (p.n + kTileM - 1) / kTileM);
        hipLaunchKernelGGL(project_tiles_kernel, grid, dim3(256), 0, stream, p);
    }
    hipLaunchKernelGGL(post_norm_kernel, dim3(p.n), dim3(256), 0, stream, p);
    return hipGetLastError();
}

} // namespace pcl

extern "C" int pcl_attention_output(pcl_context *ctx, const float *attended, int64_t n,
                                    int64_t in, const float *weights, int64_t out,
                                    const float *post_scale, float epsilon,
                                    const float *residual, float *projected, float *result)
{
    if (!ctx || !attended || !weights || !post_scale || !residual || !projected || !result)
        return PCL_INVALID_SHAPE;
    // sizes keep every grid below 2^31 work-items (post-norm: 256 per token)
    if (n <= 0 || in <= 0 || out <= 0 || n > (1 << 22) || in > (1 << 20) || out > (1 << 20))
        return PCL_INVALID_SHAPE;
    if (!(epsilon > 0.0f) || !__builtin_isfinite(epsilon))
        return PCL_INVALID_PARAMETER;
    (void)hipSetDevice(ctx->device);
    pcl::BlockParams p{};
    p.x = attended;
    p.w = weights;
    p.proj = projected;
    p.scale = post_scale;
    p.res = residual;
    p.result = result;
    p.n = (int)n;
    p.in = (int)in;
    p.out = (int)out;
    p.eps = epsilon;
    p.err = ctx->err;
    const hipError_t e = pcl::launch_output_block(p, ctx->stream);
    if (e != hipSuccess) {
        std::fprintf(stderr, "pcl_attention_output: launch: %s\n", hipGetErrorString(e));
        return PCL_NON_FINITE_VALUE;
    }
    return PCL_OK;
}

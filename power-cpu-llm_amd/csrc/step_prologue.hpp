// The head transform of one token (the engine's HeadTransform::prepare,
// src/engine/attention.rs:102-156) as device functions: the arithmetic of
// head_transform.hip, which calls the same functions, and the prologue a
// decode kernel runs when a one-token step's transform is folded into its
// launch (Params::sq).
//
// Per row of D values (p9_ref_rms_norm, src/kernels/portable/reference.rs:
// 11-33, then p9_ref_rope, reference.rs:277-318):
//   sum = sequential f64 sum of f64(x_j)^2, j ascending;
//   inv = 1 / sqrt(sum / D + f64(eps))            (f64, correctly rounded);
//   y_j = f32(f64(x_j) * inv), times scale_j in f32 for Q and K;
//   Q and K rotate pairs (j, j + D/2) by the position's (s, c):
//   y_j' = y_j*c - y_{j+h}*s,  y_{j+h}' = y_{j+h}*c + y_j*s   (f32, unfused).
#pragma once

#include "attention_device.hpp"

namespace pcl {

// The norm's inverse for a row of D floats in LDS (16-byte aligned), by the
// calling lane: the sum runs in order while the next 16 values' reads are in
// flight, so the chain of D dependent f64 adds is the time, not D LDS round
// trips. Fully unrolled (the head-transform kernel; 3 us faster over a
// 4K-token prompt) the compiler hoists every read of the row into registers;
// COMPACT (a decode kernel's prologue, whose registers are spoken for) keeps
// two batches per iteration.
template <int D, bool COMPACT = false>
__device__ __forceinline__ double norm_inverse(const float *row, float eps)
{
    constexpr int B = D < 16 ? D : 16; // floats per batch
    static_assert(D % B == 0 && B % 4 == 0, "whole batches of whole 16-byte reads");
    f4 cur[B / 4], nxt[B / 4];
#pragma unroll
    for (int i = 0; i < B / 4; ++i)
        cur[i] = *(const f4 *)(row + 4 * i);
    double sum = 0.0;
    if constexpr (COMPACT) {
#pragma unroll 2
        for (int b = 0; b < D; b += B) {
            if (b + B < D) {
#pragma unroll
                for (int i = 0; i < B / 4; ++i)
                    nxt[i] = *(const f4 *)(row + b + B + 4 * i);
            }
#pragma unroll
            for (int i = 0; i < B / 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const double v = (double)cur[i][e];
                    sum = sum + v * v;
                }
            if (b + B < D) {
#pragma unroll
                for (int i = 0; i < B / 4; ++i)
                    cur[i] = nxt[i];
            }
        }
    } else {
#pragma unroll
        for (int b = 0; b < D; b += B) {
            if (b + B < D) {
#pragma unroll
                for (int i = 0; i < B / 4; ++i)
                    nxt[i] = *(const f4 *)(row + b + B + 4 * i);
            }
#pragma unroll
            for (int i = 0; i < B / 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const double v = (double)cur[i][e];
                    sum = sum + v * v;
                }
            if (b + B < D) {
#pragma unroll
                for (int i = 0; i < B / 4; ++i)
                    cur[i] = nxt[i];
            }
        }
    }
    return 1.0 / __builtin_sqrt(sum / (double)D + (double)eps);
}

// Pair (j, j + D/2) of a row with norm inverse inv: normalised, then scaled
// by (sa, sb) and rotated by (s, c) when ROT (Q and K), plain otherwise (V).
template <bool ROT>
__device__ __forceinline__ void transform_pair(float xa, float xb, double inv, float sa, float sb,
                                               float s, float c, float *ya, float *yb)
{
    float a = (float)((double)xa * inv);
    float b = (float)((double)xb * inv);
    if (ROT) {
        a = a * sa;
        b = b * sb;
        const float ac = a * c, bs = b * s;
        const float bc = b * c, as = a * s;
        a = ac - bs;
        b = bc + as;
    }
    *ya = a;
    *yb = b;
}

// Waits for the wave's LDS accesses and keeps the compiler from moving
// memory operations across (lanes of one wave exchanging data in LDS).
__device__ __forceinline__ void wave_lds_sync()
{
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// This lane's rotation pairs j = lane + 64m of the step's position: (s, c)
// and the learned scales of both halves (Q's or K's).
template <int D> struct StepRotation {
    static constexpr int H = D / 2;
    static constexpr int PAIRS = (H + 63) / 64;
    float s[PAIRS], c[PAIRS], sa[PAIRS], sb[PAIRS];

    __device__ __forceinline__ void load(const Params &p, const float *scale)
    {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int m = 0; m < PAIRS; ++m) {
            const int j = lane + 64 * m < H ? lane + 64 * m : 0;
            s[m] = ldg(p.srot + 2 * j);
            c[m] = ldg(p.srot + 2 * j + 1);
            sa[m] = ldg(scale + j);
            sb[m] = ldg(scale + j + H);
        }
    }
};

// The prepared K (KEY) or V row of KV head kh of the step's token, by one
// wave: staged through buf (D floats of LDS, 16-byte aligned) and stored at
// the step's new cache row. Whether an input or output is not finite.
template <int D, bool KEY>
__device__ __forceinline__ bool step_kv_row(const Params &p, int kh, float *buf)
{
    constexpr int H = D / 2;
    constexpr int PAIRS = StepRotation<D>::PAIRS;
    const int lane = threadIdx.x & 63;
    const float *raw = (KEY || !p.sv ? p.sk : p.sv) + (int64_t)kh * D;
    float *dst = (KEY ? p.snk : p.snv) + (int64_t)kh * D;
    // the row and (K) the rotation pairs requested together
    StepRotation<D> rot;
    f4 x[(D / 4 + 63) / 64];
#pragma unroll
    for (int k = 0; k < (D / 4 + 63) / 64; ++k)
        if (lane + 64 * k < D / 4)
            x[k] = ldg4(raw + 4 * (lane + 64 * k));
    if (KEY)
        rot.load(p, p.sks);
    bool bad = false;
#pragma unroll
    for (int k = 0; k < (D / 4 + 63) / 64; ++k)
        if (lane + 64 * k < D / 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                bad |= !is_finite(x[k][e]);
            *(f4 *)(buf + 4 * (lane + 64 * k)) = x[k];
        }
    wave_lds_sync();
    double inv = 0.0;
    if (lane == 0)
        inv = norm_inverse<D, true>(buf, p.seps);
    inv = __shfl(inv, 0);
#pragma unroll
    for (int m = 0; m < PAIRS; ++m) {
        const int j = lane + 64 * m;
        if (j >= H)
            continue;
        float a, b;
        if (KEY)
            transform_pair<true>(buf[j], buf[j + H], inv, rot.sa[m], rot.sb[m], rot.s[m],
                                 rot.c[m], &a, &b);
        else
            transform_pair<false>(buf[j], buf[j + H], inv, 0.f, 0.f, 0.f, 0.f, &a, &b);
        bad |= !is_finite(a) || !is_finite(b);
        stg(dst + j, a);
        stg(dst + j + H, b);
    }
    wave_lds_sync(); // buf is free again
    return bad;
}

// The prepared query rows of 16-row unit `unit` of KV head kh, by one wave,
// into qb (row r at qb + r * ld, 16-byte aligned): flat row unit*16 + r
// (query 0, head kh*group + row % group), pre-scaled by q_scale as the
// kernels scale a loaded query; rows past nrows are zero. With `out`, the
// prepared (unscaled) rows are also stored to the step's query output.
// issue() requests the first pieces of the rows and the rotation pairs, so
// that a caller can request other data (its first K block) behind them and
// finish() waits only for these.
template <int D> struct StepQueryRows {
    static constexpr int H = D / 2;
    static constexpr int NV = D / 4;    // 16-byte pieces per row
    static constexpr int BATCH = 8;     // pieces per lane in flight
    static constexpr int PAIRS = StepRotation<D>::PAIRS;
    f4 x[BATCH];
    StepRotation<D> rot;
    int nr; // real rows of the unit

    __device__ __forceinline__ const float *raw_row(const Params &p, int unit, int kh, int r) const
    {
        return p.sq + (int64_t)(kh * p.group + (unit * kRows + r) % p.group) * D;
    }

    // pieces i = i0 + lane + 64k (k < BATCH) of the unit's real rows
    __device__ __forceinline__ void load_batch(const Params &p, int unit, int kh, int i0)
    {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
            const int i = i0 + lane + 64 * k;
            if (i < nr * NV)
                x[k] = ldg4(raw_row(p, unit, kh, i / NV) + 4 * (i % NV));
        }
    }

    __device__ __forceinline__ bool store_batch(float *qb, int ld, int i0)
    {
        const int lane = threadIdx.x & 63;
        bool bad = false;
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
            const int i = i0 + lane + 64 * k;
            if (i < nr * NV) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    bad |= !is_finite(x[k][e]);
                *(f4 *)(qb + (i / NV) * ld + 4 * (i % NV)) = x[k];
            }
        }
        return bad;
    }

    __device__ __forceinline__ void issue(const Params &p, int unit, int kh)
    {
        const int r0 = unit * kRows;
        nr = p.nrows - r0 < kRows ? p.nrows - r0 : kRows;
        load_batch(p, unit, kh, 0);
        rot.load(p, p.sqs);
    }

    __device__ __forceinline__ bool finish(const Params &p, int unit, int kh, float *qb, int ld,
                                           bool out)
    {
        const int lane = threadIdx.x & 63;
        bool bad = store_batch(qb, ld, 0);
        // further batches (more than BATCH pieces per lane), one in flight
#pragma unroll 1
        for (int i0 = 64 * BATCH; i0 < nr * NV; i0 += 64 * BATCH) {
            load_batch(p, unit, kh, i0);
            bad |= store_batch(qb, ld, i0);
        }
        // padding rows are zero
        for (int i = nr * NV + lane; i < kRows * NV; i += 64)
            *(f4 *)(qb + (i / NV) * ld + 4 * (i % NV)) = f4{0.f, 0.f, 0.f, 0.f};
        wave_lds_sync();
        double inv = 0.0;
        if (lane < nr)
            inv = norm_inverse<D, true>(qb + lane * ld, p.seps);
        for (int r = 0; r < nr; ++r) {
            const double iv = __shfl(inv, r);
            float *row = qb + r * ld;
            float *qo = p.sqo + (int64_t)(kh * p.group + (unit * kRows + r) % p.group) * D;
#pragma unroll
            for (int m = 0; m < PAIRS; ++m) {
                const int j = lane + 64 * m;
                if (j >= H)
                    continue;
                float a, b;
                transform_pair<true>(row[j], row[j + H], iv, rot.sa[m], rot.sb[m], rot.s[m],
                                     rot.c[m], &a, &b);
                bad |= !is_finite(a) || !is_finite(b);
                if (out) {
                    stg(qo + j, a);
                    stg(qo + j + H, b);
                }
                row[j] = a * p.q_scale;
                row[j + H] = b * p.q_scale;
            }
        }
        wave_lds_sync();
        return bad;
    }
};

} // namespace pcl

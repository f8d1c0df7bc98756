// Shared device helpers for the gfx950 VNN kernels: activations, complex arithmetic,
// deterministic wave64 / workgroup reductions, launch-status plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/neurocell_hip.h"

#define NC_DEV __device__ __forceinline__

// Compiler scheduling pins: NC_PIN(x) makes x a value that must exist at this point (in a
// VGPR), NC_FENCE() keeps memory operations on their side.  Both emit no instruction.  (A
// test harness that compiles these sources for the CPU predefines them.)
#ifndef NC_PIN
#define NC_PIN(x) asm volatile("" : "+v"(x))
#define NC_FENCE() asm volatile("" ::: "memory")
#endif
// Orders LDS accesses between the lanes of one wavefront: a wavefront's LDS operations
// complete in issue order, so keeping the compiler from moving them across this point is
// enough (no s_barrier).  Every lane of the wavefront must reach it.
#ifndef NC_WAVE_SYNC
#define NC_WAVE_SYNC() asm volatile("" ::: "memory")
#endif
#define NC_WAVE 64

// Status of a launch sequence: the first failing HIP call's code, else NC_OK.
#define NC_CHECK_LAUNCH()                                  \
    do {                                                   \
        hipError_t _e = hipGetLastError();                 \
        if (_e != hipSuccess) return (int)_e;              \
    } while (0)

static inline hipStream_t nc_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------------------
// Activations (kernels_pallas.py:111-156).  `act` is one of NC_ACT_*.
// ---------------------------------------------------------------------------------------

NC_DEV float nc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// Branch-free fp32 tanh for the per-element activations (4M evaluations per config-0
// epilogue call).  |x| < 0.25: the odd Taylor series of tanh through x^9 (truncation below
// 1e-8 relative); otherwise 1 - 2 / (exp(2|x|) + 1) with the hardware exp2 and reciprocal
// (absolute error ~1e-7; exp overflows to +inf for |x| > 44 and the result saturates at 1).
NC_DEV float nc_tanh(float x) {
    const float ax = fabsf(x);
    const float x2 = x * x;
    float p = fmaf(x2, 62.0f / 2835.0f, -17.0f / 315.0f);
    p = fmaf(x2, p, 2.0f / 15.0f);
    p = fmaf(x2, p, -1.0f / 3.0f);
    const float small = fmaf(x * x2, p, x);
    const float e = __builtin_amdgcn_exp2f(ax * 2.8853900817779268f);  // exp(2|x|)
    const float big = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
    return ax < 0.25f ? small : copysignf(big, x);
}

// tanh and its derivative.  For |x| >= 0.25 the derivative is r (2 - r) with
// r = 2 / (exp(2|x|) + 1) = 1 - |tanh x|, which keeps full relative accuracy where tanh
// saturates (1 - t*t from a rounded t would cancel).
NC_DEV float nc_tanh_d(float x, float* y) {
    const float ax = fabsf(x);
    const float x2 = x * x;
    float p = fmaf(x2, 62.0f / 2835.0f, -17.0f / 315.0f);
    p = fmaf(x2, p, 2.0f / 15.0f);
    p = fmaf(x2, p, -1.0f / 3.0f);
    const float small = fmaf(x * x2, p, x);
    const float e = __builtin_amdgcn_exp2f(ax * 2.8853900817779268f);
    const float r = 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
    const bool sm = ax < 0.25f;
    *y = sm ? small : copysignf(1.0f - r, x);
    return sm ? fmaf(-small, small, 1.0f) : r * (2.0f - r);
}

NC_DEV float nc_act(float x, int act, float neg_slope) {
    switch (act) {
        case NC_ACT_TANH: return nc_tanh(x);
        case NC_ACT_SIGMOID: return nc_sigmoid(x);
        case NC_ACT_RELU: return fmaxf(x, 0.0f);
        case NC_ACT_LEAKY_RELU: return x >= 0.0f ? x : neg_slope * x;
        case NC_ACT_GELU: {
            const float c = 0.7978845608028654f;  // sqrt(2/pi)
            return 0.5f * x * (1.0f + nc_tanh(c * (x + 0.044715f * x * x * x)));
        }
        default: return x;
    }
}

// Compile-time activation: kernels are instantiated per activation so the hot loops carry
// no per-element dispatch.
template <int ACT>
NC_DEV float act_f(float x, float neg_slope) {
    if constexpr (ACT == NC_ACT_TANH) return nc_tanh(x);
    else if constexpr (ACT == NC_ACT_SIGMOID) return nc_sigmoid(x);
    else if constexpr (ACT == NC_ACT_RELU) return fmaxf(x, 0.0f);
    else if constexpr (ACT == NC_ACT_LEAKY_RELU) return x >= 0.0f ? x : neg_slope * x;
    else if constexpr (ACT == NC_ACT_GELU) {
        const float c = 0.7978845608028654f;
        return 0.5f * x * (1.0f + nc_tanh(c * (x + 0.044715f * x * x * x)));
    } else return x;
}

template <int ACT>
NC_DEV float act_fd(float x, float neg_slope, float* y) {
    if constexpr (ACT == NC_ACT_TANH) {
        return nc_tanh_d(x, y);
    } else if constexpr (ACT == NC_ACT_SIGMOID) {
        const float s = nc_sigmoid(x);
        *y = s;
        return s * (1.0f - s);
    } else if constexpr (ACT == NC_ACT_RELU) {
        *y = fmaxf(x, 0.0f);
        return x > 0.0f ? 1.0f : 0.0f;
    } else if constexpr (ACT == NC_ACT_LEAKY_RELU) {
        *y = x >= 0.0f ? x : neg_slope * x;
        return x >= 0.0f ? 1.0f : neg_slope;
    } else if constexpr (ACT == NC_ACT_GELU) {
        const float c = 0.7978845608028654f;
        const float x2 = x * x;
        const float th = nc_tanh(c * (x + 0.044715f * x2 * x));
        const float du = c * (1.0f + 3.0f * 0.044715f * x2);
        *y = 0.5f * x * (1.0f + th);
        return 0.5f * (1.0f + th) + 0.5f * x * (1.0f - th * th) * du;
    } else {
        *y = x;
        return 1.0f;
    }
}

// Runs `f.template operator()<ACT>()` for the runtime activation id (host-side dispatch).
template <class F>
inline int dispatch_act(int act, F&& f) {
    switch (act) {
        case NC_ACT_IDENTITY: return f.template operator()<NC_ACT_IDENTITY>();
        case NC_ACT_TANH: return f.template operator()<NC_ACT_TANH>();
        case NC_ACT_SIGMOID: return f.template operator()<NC_ACT_SIGMOID>();
        case NC_ACT_RELU: return f.template operator()<NC_ACT_RELU>();
        case NC_ACT_LEAKY_RELU: return f.template operator()<NC_ACT_LEAKY_RELU>();
        case NC_ACT_GELU: return f.template operator()<NC_ACT_GELU>();
        default: return NC_ERR_INVALID_ARGUMENT;
    }
}

// Value and derivative together.
NC_DEV float nc_act_d(float x, int act, float neg_slope, float* y) {
    switch (act) {
        case NC_ACT_TANH: return nc_tanh_d(x, y);
        case NC_ACT_SIGMOID: {
            float s = nc_sigmoid(x);
            *y = s;
            return s * (1.0f - s);
        }
        case NC_ACT_RELU:
            *y = fmaxf(x, 0.0f);
            return x > 0.0f ? 1.0f : 0.0f;
        case NC_ACT_LEAKY_RELU:
            *y = x >= 0.0f ? x : neg_slope * x;
            return x >= 0.0f ? 1.0f : neg_slope;
        case NC_ACT_GELU: {
            const float c = 0.7978845608028654f;
            float x2 = x * x;
            float th = nc_tanh(c * (x + 0.044715f * x2 * x));
            float du = c * (1.0f + 3.0f * 0.044715f * x2);
            *y = 0.5f * x * (1.0f + th);
            return 0.5f * (1.0f + th) + 0.5f * x * (1.0f - th * th) * du;
        }
        default:
            *y = x;
            return 1.0f;
    }
}

// ---------------------------------------------------------------------------------------
// Complex helpers (float2 = re, im)
// ---------------------------------------------------------------------------------------

typedef float2 cpx;
NC_DEV cpx cmk(float r, float i) { return make_float2(r, i); }
NC_DEV cpx cadd(cpx a, cpx b) { return make_float2(a.x + b.x, a.y + b.y); }
NC_DEV cpx csub(cpx a, cpx b) { return make_float2(a.x - b.x, a.y - b.y); }
NC_DEV cpx cmul(cpx a, cpx b) { return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x); }
// a * conj(b)
NC_DEV cpx cmulc(cpx a, cpx b) { return make_float2(a.x * b.x + a.y * b.y, a.y * b.x - a.x * b.y); }
NC_DEV cpx cconj(cpx a) { return make_float2(a.x, -a.y); }
NC_DEV cpx cscale(cpx a, float s) { return make_float2(a.x * s, a.y * s); }
NC_DEV cpx cmul_i(cpx a) { return make_float2(-a.y, a.x); }      // i * a
NC_DEV cpx cmul_negi(cpx a) { return make_float2(a.y, -a.x); }   // -i * a

// ---------------------------------------------------------------------------------------
// Deterministic reductions.  A wave64 butterfly (xor shuffles) followed by a fixed-order
// sum over the waves of the workgroup through LDS.  Every lane returns the same value.
// ---------------------------------------------------------------------------------------

NC_DEV float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, NC_WAVE);
    return v;
}

// Sums K values per thread across a workgroup of NT threads; `red` must hold K * NT/64
// floats.  Wave totals go to LDS, then thread k < K sums the NT/64 wave totals of value k in
// fixed order and publishes it.  On return vals[k] is the workgroup total in every thread.
// Contains two barriers.
template <int K, int NT>
NC_DEV void block_sum(float* vals, float* red) {
    constexpr int NW = NT / NC_WAVE;
    static_assert(NW * NC_WAVE == NT, "workgroup must be whole waves");
    const int lane = threadIdx.x & (NC_WAVE - 1);
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        float s = wave_sum(vals[k]);
        if (lane == 0) red[k * NW + wave] = s;
    }
    __syncthreads();
    if (threadIdx.x < K) {
        const int k = threadIdx.x;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) s += red[k * NW + w];
        red[K * NW + k] = s;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k) vals[k] = red[K * NW + k];
    __syncthreads();  // red may be reused right away
}

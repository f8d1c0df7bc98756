// Piece 2 on large spectral grids (an axis of 128 or 256 points; both axes in {64, 128, 256}):
// the Green's-function correlation and its Plancherel backward with workgroup-level,
// LDS-segmented transforms (nc_lfft.h).  Same operator semantics as the wavefront kernels of
// nc_spectral.hip (kernels_pallas.py:1759-1826, kernels_greens.py:240-400); spectra are
// (FH, FW/2+1) complex64 half-spectra.
//
//   k_lrfft2<FLIP>   grid (planes, column segments)  half-spectra of real planes: cell spectra
//                                                    xhat_b, filter spectra (FLIP) and the
//                                                    cotangent spectra rfft2(gz_bm)
//   k_linv_conv      grid (B*M, row segments)        z_bm = irfft2(xhat_b * ghat_m), window
//   k_lred<MC>       grid (F/256, M/MC)              one pass over rfft2(gz): per bin, the
//                                                    fixed-order sums over m (dx partials per
//                                                    direction chunk) and over b (dghat)
//   k_linv_dx        grid (B, row segments)          dx_b = irfft2(sum of the chunk partials)
//                                                    with the unshifted roll
//   k_linv_filter    grid (M, row segments)          dG_m = flip(crop(roll(irfft2(dghat_m))))
//
// The backward materialises rfft2(gz) once (B*M half-spectra in the workspace) instead of
// transforming every cotangent plane twice: at these sizes a transform costs ~2.5 MFLOP
// per plane while re-reading its spectrum costs ~0.26 MB.  No atomics: both reductions are
// fixed-order loops, so results are bit-reproducible.
#include <algorithm>

#include "nc_large.h"
#include "nc_lfft.h"

namespace {

constexpr int kNT = 256;             // workgroup size of the transform kernels
constexpr size_t kLdsMax = 163840;   // LDS per workgroup on gfx950
constexpr int kRedMC = 16;           // directions per reduction workgroup

template <int FH, int FW>
using LG = LGeo<FH, FW, kNT>;

// Row pitch (cpx) of the reverse pass's cotangent half-spectra in the workspace: SP rounded up
// to 16 cpx, so every row starts on a 128-byte line and the column passes' 16- or 32-column
// tiles move whole lines (SP = FW/2 + 1 leaves every row but one in 16 straddling lines).
template <int FH, int FW>
constexpr int spec_pitch_ws() {
    return (LG<FH, FW>::SP + 15) / 16 * 16;
}

// LDS carve-up of the transform kernels, in the order lfwd_lds_bytes / linv_lds_bytes count
// it: twiddles | exchange scratch | (forward only) packed-column staging C0 | Y or T.
struct LdsParts {
    cpx* tw;
    cpx* scr;
    cpx* c0;
    cpx* seg;
};

template <int FH, int FW, bool FWD>
NC_DEV LdsParts lds_parts(float* lds) {
    LdsParts p;
    p.tw = reinterpret_cast<cpx*>(lds);
    p.scr = p.tw + NC_TW_N;
    p.c0 = FWD ? p.scr + LG<FH, FW>::SCR : nullptr;
    p.seg = p.scr + LG<FH, FW>::SCR + (FWD ? FH : 0);
    return p;
}

// Half-spectrum of one real plane src, column segment [c0, c0 + cs), each bin through
// spec_post<POST> into o.  NP > 1: each value is the sum of NP partial planes qstride floats
// apart, in increasing order (NP == 0: nq of them).
template <int FH, int FW, bool FLIP, int POST, int NP>
NC_DEV void lplane_job(const float* __restrict__ src, int hin, int win, int c0, int cs,
                       cpx* __restrict__ o, const SpecPost& post, size_t qstride, int nq,
                       const LdsParts& P) {
    using L = LG<FH, FW>;
    lplane_rfft2<FH, FW, kNT>(
        [&](int r, int c) {
            if constexpr (FLIP) return src[(hin - 1 - r) * win + (win - 1 - c)];
            const float* a = src + r * win + c;
            float v = a[0];
            if constexpr (NP > 1) {
#pragma unroll
                for (int q = 1; q < NP; ++q) v += a[q * qstride];
            } else if constexpr (NP == 0) {
                for (int q = 1; q < nq; ++q) v += a[q * qstride];
            }
            return v;
        },
        hin, win, c0, cs,
        [&](int kh, int kw, cpx v) { o[kh * L::SP + kw] = spec_post<POST, FH, FW>(v, kh, kw, post); },
        P.seg, P.c0, P.scr, P.tw);
}

template <int FH, int FW, bool FLIP, int POST, int NP>
__global__ __launch_bounds__(kNT) void k_lrfft2(int hin, int win, int cs, size_t pstride,
                                                const float* __restrict__ x,
                                                cpx* __restrict__ out, SpecPost post,
                                                size_t qstride, int nq) {
    HIP_DYNAMIC_SHARED(float, lds)
    const LdsParts P = lds_parts<FH, FW, true>(lds);
    load_twiddles(P.tw);
    __syncthreads();
    lplane_job<FH, FW, FLIP, POST, NP>(x + (size_t)blockIdx.x * pstride, hin, win,
                                        (int)blockIdx.y * cs, cs,
                                        out + (size_t)blockIdx.x * LG<FH, FW>::F, post, qstride,
                                        nq, P);
}

// Several independent spectrum jobs (nc_plane_spectra) in one launch: block (g, segment) runs
// plane g - start[q] of the job q whose range holds g.
constexpr int kMaxLJobs = 4;
struct LJobs {
    const float* x[kMaxLJobs];
    cpx* out[kMaxLJobs];
    SpecPost post[kMaxLJobs];
    int hin[kMaxLJobs], win[kMaxLJobs], kind[kMaxLJobs];
    int start[kMaxLJobs + 1];
    int n, cs;
};
enum { kLPlain = 0, kLFlip = 1, kLAdd = 2, kLShift = 3 };

template <int FH, int FW>
__global__ __launch_bounds__(kNT) void k_lspectra(LJobs J) {
    HIP_DYNAMIC_SHARED(float, lds)
    const LdsParts P = lds_parts<FH, FW, true>(lds);
    load_twiddles(P.tw);
    __syncthreads();
    const int g = blockIdx.x;
    int q = 0;
    while (q + 1 < J.n && g >= J.start[q + 1]) ++q;
    const int i = g - J.start[q], hin = J.hin[q], win = J.win[q];
    const float* src = J.x[q] + (size_t)i * hin * win;
    cpx* o = J.out[q] + (size_t)i * LG<FH, FW>::F;
    const int c0 = (int)blockIdx.y * J.cs;
    switch (J.kind[q]) {
        case kLFlip:
            lplane_job<FH, FW, true, kPostNone, 1>(src, hin, win, c0, J.cs, o, J.post[q], 0, 1, P);
            break;
        case kLAdd:
            lplane_job<FH, FW, false, kPostAdd, 1>(src, hin, win, c0, J.cs, o, J.post[q], 0, 1, P);
            break;
        case kLShift:
            lplane_job<FH, FW, false, kPostShift, 1>(src, hin, win, c0, J.cs, o, J.post[q], 0, 1,
                                                     P);
            break;
        default:
            lplane_job<FH, FW, false, kPostNone, 1>(src, hin, win, c0, J.cs, o, J.post[q], 0, 1,
                                                    P);
    }
}

// Packed column value of a half-spectrum at (kh, kw): DC + i*Nyquist for kw == 0.
template <int FW, class S>
NC_DEV cpx packed_at(S s, int kh, int kw) {
    constexpr int SP = FW / 2 + 1;
    if (kw == 0) return cadd(s(kh * SP), cmul_i(s(kh * SP + FW / 2)));
    return s(kh * SP + kw);
}

// Forward correlation: plane g = b*M + m, output rows [i0, i0 + rs) of the hout x wout window
// read from row ph, column pw of irfft2(xhat_b * ghat_m).
template <int FH, int FW>
__global__ __launch_bounds__(kNT) void k_linv_conv(int M, int hout, int wout, int ph, int pw,
                                                   int rs, const cpx* __restrict__ xhat,
                                                   const cpx* __restrict__ ghat,
                                                   float* __restrict__ z) {
    using L = LG<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    const LdsParts P = lds_parts<FH, FW, false>(lds);
    load_twiddles(P.tw);
    __syncthreads();
    const int g = blockIdx.x, b = g / M, m = g - b * M;
    const int i0 = blockIdx.y * rs, rows = min(rs, hout - i0);
    const cpx* X = xhat + (size_t)b * L::F;
    const cpx* G = ghat + (size_t)m * L::F;
    float* zo = z + (size_t)g * hout * wout + (size_t)i0 * wout;
    lplane_irfft2<FH, FW, kNT>(
        [&](int kh, int kw) {
            return packed_at<FW>([&](int e) { return cmul(X[e], G[e]); }, kh, kw);
        },
        (ph + i0) & (FH - 1), rows, pw, wout, 1.0f / (float)(FH * FW),
        [&](int i, int j, float v) { zo[i * wout + j] = v; }, P.seg, P.scr, P.tw);
}

// ---------------------------------------------------------------------------------------
// Two-pass transforms for many planes (the B*M correlation planes and cotangent planes of
// configs 2 and 3): one kernel per axis, the intermediate in HBM, so each kernel keeps ~37 KB
// of LDS (four workgroups per CU) instead of one plane's whole segment (one per CU), and no
// pass is repeated per segment.  Same transforms and bin order as lplane_irfft2 /
// lplane_rfft2; the row pass of the inverse applies the same output window.
// ---------------------------------------------------------------------------------------

// Inverse column pass: packed columns [blockIdx.x * CPW, +CPW) (column 0: DC + i*Nyquist) of
// plane g's spectrum S_g, inverse over kh, rows i = (kh - row0) mod FH < hout kept:
// T[(g * hout + i) * NC + kw], grid (column tiles, g).  SRC 0, the correlation:
// S_g = A_b * B_m for g = b*n + m; SRC 1, the dx spectra: S_g = the sum of the n chunk
// partials A[c * cstride + g * F].
enum { kSrcProduct = 0, kSrcChunks = 1 };

template <int FH, int FW, int SRC>
__global__ __launch_bounds__(kNT) void k_linv_cols(int n, size_t cstride, int hout, int row0,
                                                   const cpx* __restrict__ A,
                                                   const cpx* __restrict__ Bm,
                                                   cpx* __restrict__ T) {
    using L = LG<FH, FW>;
    constexpr int EH = L::GH::E, GH = L::GH::G, CPW = kNT / GH;
    __shared__ cpx tw[NC_TW_N];
    __shared__ cpx scr[CPW * L::SCR_HS];
    load_twiddles(tw);
    __syncthreads();
    const int tid = threadIdx.x, g = tid % CPW, t = tid / CPW;
    const int kw = blockIdx.x * CPW + g, plane = blockIdx.y;
    cpx v[EH];
    if constexpr (SRC == kSrcProduct) {
        const int b = plane / n, m = plane - b * n;
        const cpx* X = A + (size_t)b * L::F;
        const cpx* G = Bm + (size_t)m * L::F;
#pragma unroll
        for (int n1 = 0; n1 < EH; ++n1)
            v[n1] = packed_at<FW>([&](int e) { return cmul(X[e], G[e]); }, t + GH * n1, kw);
    } else {
        const cpx* src = A + (size_t)plane * L::F;
#pragma unroll
        for (int n1 = 0; n1 < EH; ++n1)
            v[n1] = packed_at<FW>(
                [&](int e) {
                    cpx s = src[e];
                    for (int c = 1; c < n; ++c) s = cadd(s, src[c * cstride + e]);
                    return s;
                },
                t + GH * n1, kw);
    }
    cpx* sc = scr + g * L::SCR_HS;
    gfft_stage1<FH, true>(v, t, sc, tw);
    __syncthreads();
    gfft_stage2<FH, true>(v, t, sc);
    cpx* To = T + (size_t)plane * hout * L::NC + kw;
#pragma unroll
    for (int s = 0; s < EH; ++s) {
        const int i = (L::GH::bin(t, s) - row0) & (FH - 1);
        if (i < hout) To[(size_t)i * L::NC] = v[s];
    }
}

// Inverse row pass: rows (2p, 2p + 1) of T as one complex transform, p in
// [blockIdx.x * PPW, +PPW); output columns j = (c - col0) mod FW < wout, times scale.
// STATS: the workgroup also forms its band's statistics, the band being its output rows
// [2 PPW blockIdx.x, +2 PPW) of the plane: the sum and the centred sum of squares about the
// band mean, both as fixed-order workgroup sums, at stats[plane * nbands + band] and
// stats[nplanes * nbands + plane * nbands + band] (the tile-statistics layout (2, B*M, T) of
// the tiled epilogue, with bands for tiles).
template <int FH, int FW, bool STATS = false>
__global__ __launch_bounds__(kNT) void k_linv_rows(int hout, int wout, int col0, float scale,
                                                   const cpx* __restrict__ T,
                                                   float* __restrict__ z,
                                                   float* __restrict__ stats) {
    using L = LG<FH, FW>;
    constexpr int EW = L::GW::E, GW = L::GW::G, PPW = kNT / GW, NC = L::NC;
    __shared__ cpx tw[NC_TW_N];
    __shared__ cpx scr[PPW * L::GW::SCR];
    load_twiddles(tw);
    __syncthreads();
    const int tid = threadIdx.x, g = tid / GW, t = tid % GW, plane = blockIdx.y;
    const int p = blockIdx.x * PPW + g, npairs = (hout + 1) >> 1;
    const bool on = p < npairs;
    const int ia = 2 * p, ib = 2 * p + 1;
    const bool hasb = ib < hout;
    const cpx* ta = T + ((size_t)plane * hout + (on ? ia : 0)) * NC;
    const cpx* tb = T + ((size_t)plane * hout + (on && hasb ? ib : (on ? ia : 0))) * NC;
    const float bs = hasb ? 1.f : 0.f;
    cpx v[EW];
#pragma unroll
    for (int n1 = 0; n1 < EW; ++n1) {
        const int k = t + GW * n1;
        cpx a, bb;
        if (n1 < EW / 2) {  // k < FW/2
            if (k == 0) {
                a = cmk(ta[0].x, 0.f);
                bb = cmk(tb[0].x, 0.f);
            } else {
                a = ta[k];
                bb = tb[k];
            }
        } else {  // k >= FW/2
            if (k == FW / 2) {
                a = cmk(ta[0].y, 0.f);
                bb = cmk(tb[0].y, 0.f);
            } else {
                a = cconj(ta[FW - k]);
                bb = cconj(tb[FW - k]);
            }
        }
        v[n1] = cadd(a, cmul_i(cscale(bb, bs)));
    }
    cpx* sc = scr + g * L::GW::SCR;
    gfft_stage1<FW, true>(v, t, sc, tw);
    __syncthreads();
    gfft_stage2<FW, true>(v, t, sc);
    if constexpr (STATS) {
        __shared__ float red[kNT / 64 + 1];
        float s1 = 0.f;
#pragma unroll
        for (int s = 0; s < EW; ++s) {
            const int j = (L::GW::bin(t, s) - col0) & (FW - 1);
            if (on && j < wout) s1 += v[s].x * scale + (hasb ? v[s].y * scale : 0.f);
        }
        block_sum<1, kNT>(&s1, red);
        const int rows = min(2 * PPW, hout - 2 * PPW * (int)blockIdx.x);
        const float mu = s1 / (float)(rows * wout);
        float m2 = 0.f;
#pragma unroll
        for (int s = 0; s < EW; ++s) {
            const int j = (L::GW::bin(t, s) - col0) & (FW - 1);
            if (on && j < wout) {
                const float da = v[s].x * scale - mu, db = hasb ? v[s].y * scale - mu : 0.f;
                m2 += da * da + db * db;
            }
        }
        block_sum<1, kNT>(&m2, red);
        if (threadIdx.x == 0) {
            const size_t o = (size_t)plane * gridDim.x + blockIdx.x;
            stats[o] = s1;
            stats[(size_t)gridDim.y * gridDim.x + o] = m2;
        }
    }
    if (!on) return;
    float* za = z + ((size_t)plane * hout + ia) * wout;
#pragma unroll
    for (int s = 0; s < EW; ++s) {
        const int j = (L::GW::bin(t, s) - col0) & (FW - 1);
        if (j < wout) {
            za[j] = v[s].x * scale;
            if (hasb) za[wout + j] = v[s].y * scale;
        }
    }
}

// Forward row pass of real planes (plane g at x + g * pstride, hin x win at the grid origin,
// each value the sum of nq partial planes qstride floats apart, in increasing order): rows
// (2p, 2p + 1) as one complex transform, split into the two rows' half-spectra, written as
// rows 2p, 2p + 1 of the plane's (FH, PITCH) half-spectrum region of U (bins kw <= FW/2 of a
// row; PITCH >= SP).  Rows >= hin are not written (the column pass reads them as zeros).
template <int FH, int FW, int PITCH = LG<FH, FW>::SP>
__global__ __launch_bounds__(kNT) void k_lrfft_rows(int hin, int win, size_t pstride, int nq,
                                                    size_t qstride, const float* __restrict__ x,
                                                    cpx* __restrict__ U) {
    using L = LG<FH, FW>;
    constexpr int EW = L::GW::E, GW = L::GW::G, PPW = kNT / GW, SP = PITCH;
    __shared__ cpx tw[NC_TW_N];
    __shared__ cpx scr[PPW * L::GW::SCR];
    load_twiddles(tw);
    __syncthreads();
    const int tid = threadIdx.x, g = tid / GW, t = tid % GW, plane = blockIdx.y;
    const int p = blockIdx.x * PPW + g, npairs = (hin + 1) >> 1;
    const bool on = p < npairs;
    const int ra = 2 * p, rb = 2 * p + 1;
    const bool hasb = on && rb < hin;
    const float* xa = x + (size_t)plane * pstride + (size_t)(on ? ra : 0) * win;
    const float* xb = x + (size_t)plane * pstride + (size_t)(hasb ? rb : 0) * win;
    cpx v[EW];
#pragma unroll
    for (int n1 = 0; n1 < EW; ++n1) {
        const int c = t + GW * n1;
        float a = 0.f, b = 0.f;
        if (on && c < win) {
            a = xa[c];
            for (int q = 1; q < nq; ++q) a += xa[q * qstride + c];
            if (hasb) {
                b = xb[c];
                for (int q = 1; q < nq; ++q) b += xb[q * qstride + c];
            }
        }
        v[n1] = cmk(a, b);
    }
    cpx* sc = scr + g * L::GW::SCR;
    gfft_stage1<FW, false>(v, t, sc, tw);
    __syncthreads();
    gfft_stage2<FW, false>(v, t, sc);
    __syncthreads();  // the stage-2 reads of the scratch are done: it holds Z for the split
#pragma unroll
    for (int s = 0; s < EW; ++s) sc[L::GW::bin(t, s)] = v[s];
    __syncthreads();
    if (!on) return;
    cpx* ua = U + (size_t)plane * FH * SP + (size_t)ra * SP;
#pragma unroll
    for (int s = 0; s < EW; ++s) {
        const int k = L::GW::bin(t, s);
        if (k <= FW / 2) {
            // A[k] = (Z[k] + conj Z[-k]) / 2, B[k] = -i (Z[k] - conj Z[-k]) / 2
            const cpx zk = v[s], zm = sc[(FW - k) & (FW - 1)];
            ua[k] = cmk(0.5f * (zk.x + zm.x), 0.5f * (zk.y - zm.y));
            if (hasb) ua[SP + k] = cmk(0.5f * (zk.y + zm.y), 0.5f * (zm.x - zk.x));
        }
    }
}

// The workgroup's band of gz (rows [r0, r0 + nr) of plane g, pixel offset p0 = r0 * win) into
// LDS, row-major with pitch win: coalesced loads of z, gy and the per-pixel parameters, four
// consecutive pixels per 16-byte load with VEC.
template <int ACT, bool VEC, int NT>
NC_DEV void epi_gz_band(float* S, const nc_epi_gz& e, size_t zo, size_t go, int p0, int n,
                        float mu, float r, float c1, float c2) {
    const int tid = threadIdx.x;
    if constexpr (VEC) {
        const float4* z4 = reinterpret_cast<const float4*>(e.z + zo + p0);
        const float4* g4 = reinterpret_cast<const float4*>(e.gy + go + p0);
        const float4* w4 = reinterpret_cast<const float4*>(e.w_eff + p0);
        const float4* s4 = reinterpret_cast<const float4*>(e.s_eff + p0);
        const float4* b4 = reinterpret_cast<const float4*>(e.b_roi + p0);
#pragma unroll 2
        for (int i = tid; i < (n >> 2); i += NT) {
            const float4 zv = z4[i], gv = g4[i], wv = w4[i], sv = s4[i], bv = b4[i];
            const float zz[4] = {zv.x, zv.y, zv.z, zv.w}, gg[4] = {gv.x, gv.y, gv.z, gv.w};
            const float ww[4] = {wv.x, wv.y, wv.z, wv.w}, ss[4] = {sv.x, sv.y, sv.z, sv.w};
            const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
            float o[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float zn = (zz[k] - mu) * r;
                float a;
                const float da = act_fd<ACT>(zn + bb[k], e.neg_slope, &a);
                const float gn = gg[k] * (ww[k] + ss[k] * da);
                o[k] = r * (gn - c1 - zn * c2);
            }
            reinterpret_cast<float4*>(S)[i] = make_float4(o[0], o[1], o[2], o[3]);
        }
    } else {
        for (int i = tid; i < n; i += NT) {
            const float zn = (e.z[zo + p0 + i] - mu) * r;
            float a;
            const float da = act_fd<ACT>(zn + e.b_roi[p0 + i], e.neg_slope, &a);
            const float gn = e.gy[go + p0 + i] * (e.w_eff[p0 + i] + e.s_eff[p0 + i] * da);
            S[i] = r * (gn - c1 - zn * c2);
        }
    }
}

// k_lrfft_rows over the cotangent planes of the tiled epilogue backward, formed as they are
// read (nc_epi_gz; each workgroup stages its band of rows in LDS first): plane g = b*M + m's
// value at pixel p is
//   rstd_g * (gy_b[p] * (w[p] + s[p] * act'(zhat + b_roi[p])) - c1 - zhat * c2),
//   zhat = (z_g[p] - mean_g) * rstd_g,
// with (c1, c2) the plane's tile partials summed by the workgroup in the order the
// epilogue's own second stage sums them, so the values equal the gz it would have stored.
template <int FH, int FW, int PITCH>
__global__ __launch_bounds__(kNT) void k_lrfft_rows_epi(int M, int hin, int win, int vec,
                                                        nc_epi_gz e, cpx* __restrict__ U) {
    using L = LG<FH, FW>;
    constexpr int EW = L::GW::E, GW = L::GW::G, PPW = kNT / GW, SP = PITCH;
    static_assert((size_t)2 * PPW * FW * sizeof(float) <= PPW * L::GW::SCR * sizeof(cpx),
                  "the band staging fits the exchange scratch");
    __shared__ cpx tw[NC_TW_N];
    __shared__ cpx scr[PPW * L::GW::SCR];  // first the band's gz staging, then the exchange
    __shared__ float red[2 * (kNT / 64) + 2];
    float* S = reinterpret_cast<float*>(scr);
    load_twiddles(tw);
    const int tid = threadIdx.x, g = tid / GW, t = tid % GW, plane = blockIdx.y;
    const int b = plane / M, N = hin * win;
    const size_t BMT = (size_t)gridDim.y * e.n_tiles;
    float c[2] = {0.f, 0.f};
    for (int u = tid; u < e.n_tiles; u += kNT) {
        c[0] += e.cpart[(size_t)plane * e.n_tiles + u];
        c[1] += e.cpart[BMT + (size_t)plane * e.n_tiles + u];
    }
    block_sum<2, kNT>(c, red);  // its barriers also order the twiddle copy
    const float c1 = c[0] / (float)N, c2 = c[1] / (float)N;
    const float mu = e.mean[plane], r = e.rstd[plane];
    const int r0 = blockIdx.x * 2 * PPW, nr = min(2 * PPW, hin - r0);
    const size_t zo = (size_t)plane * N, go = (size_t)b * N;
#define NC_BAND(A_)                                                                            \
    (vec ? epi_gz_band<A_, true, kNT>(S, e, zo, go, r0 * win, nr * win, mu, r, c1, c2)        \
         : epi_gz_band<A_, false, kNT>(S, e, zo, go, r0 * win, nr * win, mu, r, c1, c2))
    switch (e.act) {  // uniform over the launch
        case NC_ACT_TANH: NC_BAND(NC_ACT_TANH); break;
        case NC_ACT_SIGMOID: NC_BAND(NC_ACT_SIGMOID); break;
        case NC_ACT_RELU: NC_BAND(NC_ACT_RELU); break;
        case NC_ACT_LEAKY_RELU: NC_BAND(NC_ACT_LEAKY_RELU); break;
        case NC_ACT_GELU: NC_BAND(NC_ACT_GELU); break;
        default: NC_BAND(NC_ACT_IDENTITY);
    }
#undef NC_BAND
    __syncthreads();
    const int p = blockIdx.x * PPW + g, npairs = (hin + 1) >> 1;
    const bool on = p < npairs;
    const int ra = 2 * p, rb = 2 * p + 1;
    const bool hasb = on && rb < hin;
    const float* sa = S + (on ? ra - r0 : 0) * win;
    const float* sb = S + (hasb ? rb - r0 : 0) * win;
    cpx v[EW];
#pragma unroll
    for (int n1 = 0; n1 < EW; ++n1) {
        const int col = t + GW * n1;
        const bool in = on && col < win;
        v[n1] = cmk(in ? sa[col] : 0.f, in && hasb ? sb[col] : 0.f);
    }
    __syncthreads();  // the staging is rewritten by the exchange
    cpx* sc = scr + g * L::GW::SCR;
    gfft_stage1<FW, false>(v, t, sc, tw);
    __syncthreads();
    gfft_stage2<FW, false>(v, t, sc);
    __syncthreads();  // the stage-2 reads of the scratch are done: it holds Z for the split
#pragma unroll
    for (int s = 0; s < EW; ++s) sc[L::GW::bin(t, s)] = v[s];
    __syncthreads();
    if (!on) return;
    cpx* ua = U + (size_t)plane * FH * SP + (size_t)ra * SP;
#pragma unroll
    for (int s = 0; s < EW; ++s) {
        const int k = L::GW::bin(t, s);
        if (k <= FW / 2) {
            const cpx zk = v[s], zm = sc[(FW - k) & (FW - 1)];
            ua[k] = cmk(0.5f * (zk.x + zm.x), 0.5f * (zk.y - zm.y));
            if (hasb) ua[SP + k] = cmk(0.5f * (zk.y + zm.y), 0.5f * (zm.x - zk.x));
        }
    }
}

// Forward column pass, in place: columns [blockIdx.x * CPW, +CPW) (< SP) of plane g's
// row-transformed rows r < hin (rows >= hin are zero), transformed over r into every bin kh,
// plus add[kh * SP + kw] when add is given (one spectrum for every plane).  A column belongs
// to one thread group of one workgroup, and the workgroup's barrier orders all its reads
// before its writes.  Planes are FH rows of PITCH cpx apart.
template <int FH, int FW, int PITCH = LG<FH, FW>::SP>
__global__ __launch_bounds__(kNT) void k_lrfft_cols(int hin, const cpx* __restrict__ add,
                                                    cpx* __restrict__ U) {
    using L = LG<FH, FW>;
    constexpr int EH = L::GH::E, GH = L::GH::G, CPW = kNT / GH, SP = L::SP;
    __shared__ cpx tw[NC_TW_N];
    __shared__ cpx scr[CPW * L::SCR_HS];
    load_twiddles(tw);
    __syncthreads();
    const int tid = threadIdx.x, g = tid % CPW, t = tid / CPW;
    const int kw = blockIdx.x * CPW + g;
    const bool on = kw < SP;
    cpx* col = U + (size_t)blockIdx.y * FH * PITCH + (on ? kw : 0);
    cpx v[EH];
#pragma unroll
    for (int n1 = 0; n1 < EH; ++n1) {
        const int r = t + GH * n1;
        v[n1] = on && r < hin ? col[(size_t)r * PITCH] : cmk(0.f, 0.f);
    }
    cpx* sc = scr + g * L::SCR_HS;
    gfft_stage1<FH, false>(v, t, sc, tw);
    __syncthreads();
    gfft_stage2<FH, false>(v, t, sc);
    if (!on) return;
#pragma unroll
    for (int s = 0; s < EH; ++s) {
        const int kh = L::GH::bin(t, s);
        col[(size_t)kh * PITCH] = add ? cadd(v[s], add[kh * SP + kw]) : v[s];
    }
}

// Both reductions of the backward in one pass over the cotangent spectra sp (B, M, FH rows of
// sp_pitch cpx, the first spw of each row the bins kw = 0 .. FW/2):
//   dxpart[c][b] = sum over the chunk's directions m of sp_bm * conj(ghat_m)   (need_dx)
//   dghat[m]     = (+=) sum over b of sp_bm * conj(xhat_b)  (conjugated when conj_out)
//   ssum[m]      = (+=, sum_acc) sum over b of sp_bm, the spectrum of sum_b gz_bm  (with ssum)
// Thread = one bin; directions m0 .. m0+MC-1 of chunk c = blockIdx.y; b in increasing order
// over sample slice blockIdx.z, whose sums go to row blockIdx.z of dghat / ssum (M*F each).
template <int MC>
__global__ __launch_bounds__(256) void k_lred(int B, int M, int F, int spw, int sp_pitch,
                                              int need_dx, const cpx* __restrict__ sp,
                                              const cpx* __restrict__ xhat,
                                              const cpx* __restrict__ ghat,
                                              cpx* __restrict__ dxpart, cpx* __restrict__ dghat,
                                              int accumulate, int conj_out,
                                              cpx* __restrict__ ssum, int sum_acc) {
    // threads walk sp's rows (pitch sp_pitch, so a wavefront's loads are whole aligned lines);
    // the pitch's padding columns have no bin
    const int es = blockIdx.x * blockDim.x + threadIdx.x;
    const int kh = es / sp_pitch, kw = es - kh * sp_pitch;
    if (kw >= spw || kh >= F / spw) return;
    const int e = kh * spw + kw;                     // the bin in the other arrays
    const size_t FP = (size_t)(F / spw) * sp_pitch;  // sp's plane stride
    const int m0 = blockIdx.y * MC;
    const int nm = min(MC, M - m0);
    // sample slice z = blockIdx.z: b in [b0, b1), its sums into row z of dghat / ssum
    const int bc = (B + gridDim.z - 1) / gridDim.z, b0 = blockIdx.z * bc, b1 = min(B, b0 + bc);
    dghat += (size_t)blockIdx.z * M * F;
    if (ssum) ssum += (size_t)blockIdx.z * M * F;
    cpx G[MC], acc[MC], sacc[MC];
#pragma unroll
    for (int q = 0; q < MC; ++q) {
        G[q] = ghat[(size_t)(m0 + min(q, nm - 1)) * F + e];
        acc[q] = cmk(0.f, 0.f);
        sacc[q] = cmk(0.f, 0.f);
    }
    for (int b = b0; b < b1; ++b) {
        const cpx X = xhat[(size_t)b * F + e];
        const cpx* s = sp + ((size_t)b * M + m0) * FP + es;
        cpx v[MC];
#pragma unroll
        for (int q = 0; q < MC; ++q) v[q] = s[(size_t)min(q, nm - 1) * FP];
        cpx d = cmk(0.f, 0.f);
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            if (q < nm) {
                d = cadd(d, cmulc(v[q], G[q]));
                acc[q] = cadd(acc[q], cmulc(v[q], X));
                sacc[q] = cadd(sacc[q], v[q]);
            }
        }
        if (need_dx) dxpart[((size_t)blockIdx.y * B + b) * F + e] = d;
    }
#pragma unroll
    for (int q = 0; q < MC; ++q) {
        if (q < nm) {
            const cpx v = conj_out ? cconj(acc[q]) : acc[q];
            cpx* o = dghat + (size_t)(m0 + q) * F + e;
            *o = accumulate ? cadd(*o, v) : v;
            if (ssum) {
                cpx* so = ssum + (size_t)(m0 + q) * F + e;
                *so = sum_acc ? cadd(*so, sacc[q]) : sacc[q];
            }
        }
    }
}

// dx, last stage: sample b's spectrum is the fixed-order sum of its nchunk partials; the
// inverse applies the unshifted roll (kernels_pallas.py:1798-1812): rows from (FH - ph) mod FH,
// columns from (FW - pw) mod FW, hin x win kept; rows [i0, i0 + rs) here.
// NCH > 0: a compile-time count of nchunk, so the partials' loads are issued together.
template <int FH, int FW, int NCH>
__global__ __launch_bounds__(kNT) void k_linv_dx(int B, int nchunk, int hin, int win, int ph,
                                                 int pw, int rs, const cpx* __restrict__ part,
                                                 float* __restrict__ dx) {
    using L = LG<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    const LdsParts P = lds_parts<FH, FW, false>(lds);
    load_twiddles(P.tw);
    __syncthreads();
    const int b = blockIdx.x;
    const int i0 = blockIdx.y * rs, rows = min(rs, hin - i0);
    const cpx* src = part + (size_t)b * L::F;
    const size_t cstride = (size_t)B * L::F;
    float* o = dx + (size_t)b * hin * win + (size_t)i0 * win;
    lplane_irfft2<FH, FW, kNT>(
        [&](int kh, int kw) {
            return packed_at<FW>(
                [&](int e) {
                    cpx s = src[e];
                    if constexpr (NCH > 0) {
#pragma unroll
                        for (int c = 1; c < NCH; ++c) s = cadd(s, src[c * cstride + e]);
                    } else {
                        for (int c = 1; c < nchunk; ++c) s = cadd(s, src[c * cstride + e]);
                    }
                    return s;
                },
                kh, kw);
        },
        ((FH - ph) + i0) & (FH - 1), rows, (FW - pw) & (FW - 1), win, 1.0f / (float)(FH * FW),
        [&](int i, int j, float v) { o[i * win + j] = v; }, P.seg, P.scr, P.tw);
}

// Filter spectrum backward (kernels_pallas.py:1558-1579): dG_m = flip(crop(roll(irfft2(.)))),
// output rows [i0, i0 + rs) of the kh x kw crop.
template <int FH, int FW>
__global__ __launch_bounds__(kNT) void k_linv_filter(int kh, int kw, int shift_h, int shift_w,
                                                     int rs, const cpx* __restrict__ dghat,
                                                     float* __restrict__ gfilt, int accumulate,
                                                     int conj_in) {
    using L = LG<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    const LdsParts P = lds_parts<FH, FW, false>(lds);
    load_twiddles(P.tw);
    __syncthreads();
    const int m = blockIdx.x;
    const int i0 = blockIdx.y * rs, rows = min(rs, kh - i0);
    const cpx* d = dghat + (size_t)m * L::F;
    float* out = gfilt + (size_t)m * kh * kw;
    const int row0 = (FH - (shift_h % FH)) & (FH - 1);
    const int col0 = (FW - (shift_w % FW)) & (FW - 1);
    lplane_irfft2<FH, FW, kNT>(
        [&](int a, int c) {
            return packed_at<FW>(
                [&](int e) { return conj_in ? cconj(d[e]) : d[e]; }, a, c);
        },
        (row0 + i0) & (FH - 1), rows, col0, kw, 1.0f / (float)(FH * FW),
        [&](int i, int j, float v) {
            float* o = out + (kh - 1 - (i0 + i)) * kw + (kw - 1 - j);
            *o = accumulate ? *o + v : v;
        },
        P.seg, P.scr, P.tw);
}

// ----------------------------------------------------------------------------------------
// Launch plumbing
// ----------------------------------------------------------------------------------------

template <class K>
void set_lds(K kernel, size_t bytes) {
    if (bytes > 65536)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

// Packed columns per forward segment: the widest power-of-two share of FW/2 whose pair
// buffer fits in LDS.
template <int FH, int FW>
int fwd_cols(int hin) {
    int cs = LG<FH, FW>::NC;
    while (cs > 1 && lfwd_lds_bytes<FH, FW, kNT>(hin, cs) > kLdsMax) cs >>= 1;
    return cs;
}

// Output rows per inverse segment: rows split evenly into the fewest segments that fit.
template <int FH, int FW>
int inv_rows(int rows) {
    for (int n = 1;; ++n) {
        const int rs = (rows + n - 1) / n;
        if (linv_lds_bytes<FH, FW, kNT>(rs) <= kLdsMax || rs == 1) return rs;
    }
}

template <int FH, int FW, bool FLIP, int POST, int NP>
void rfft2_launch_np(hipStream_t st, dim3 grid, size_t lds, int hin, int win, int cs,
                     size_t pstride, const float* x, cpx* out, const SpecPost& post,
                     size_t qstride, int nq) {
    set_lds(k_lrfft2<FH, FW, FLIP, POST, NP>, lds);
    hipLaunchKernelGGL((k_lrfft2<FH, FW, FLIP, POST, NP>), grid, dim3(kNT), lds, st, hin, win,
                       cs, pstride, x, out, post, qstride, nq);
}

template <int FH, int FW, bool FLIP, int POST>
void rfft2_launch(hipStream_t st, dim3 grid, size_t lds, int hin, int win, int cs, size_t pstride,
                  const float* x, cpx* out, const SpecPost& post, size_t qstride, int nq) {
    if (FLIP || nq == 1)
        rfft2_launch_np<FH, FW, FLIP, POST, 1>(st, grid, lds, hin, win, cs, pstride, x, out, post,
                                               0, 1);
    else if (nq == 4)
        rfft2_launch_np<FH, FW, false, POST, 4>(st, grid, lds, hin, win, cs, pstride, x, out,
                                                post, qstride, 4);
    else
        rfft2_launch_np<FH, FW, false, POST, 0>(st, grid, lds, hin, win, cs, pstride, x, out,
                                                post, qstride, nq);
}

// Half-spectra of nplanes real planes, each bin through spec_post<post_kind> (flip: the filter
// spectra, no post-operation).
template <int FH, int FW>
int rfft2_planes(hipStream_t st, int nplanes, int hin, int win, size_t pstride, bool flip,
                 const float* x, cpx* out, int post_kind = kPostNone,
                 const SpecPost& post = SpecPost{}, int nq = 1, size_t qstride = 0) {
    int cs = fwd_cols<FH, FW>(hin);
    // few planes: more column segments (the row pass repeats per segment) to fill the CUs
    while (cs > 8 && (size_t)nplanes * (LG<FH, FW>::NC / cs) < 256) cs >>= 1;
    const size_t lds = lfwd_lds_bytes<FH, FW, kNT>(hin, cs);
    if (lds > kLdsMax) return NC_ERR_UNSUPPORTED;
    const dim3 grid(nplanes, LG<FH, FW>::NC / cs);
    if (flip)
        rfft2_launch<FH, FW, true, kPostNone>(st, grid, lds, hin, win, cs, pstride, x, out, post,
                                              qstride, nq);
    else if (post_kind == kPostAdd)
        rfft2_launch<FH, FW, false, kPostAdd>(st, grid, lds, hin, win, cs, pstride, x, out, post,
                                              qstride, nq);
    else if (post_kind == kPostShift)
        rfft2_launch<FH, FW, false, kPostShift>(st, grid, lds, hin, win, cs, pstride, x, out,
                                                post, qstride, nq);
    else
        rfft2_launch<FH, FW, false, kPostNone>(st, grid, lds, hin, win, cs, pstride, x, out, post,
                                               qstride, nq);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int spec_fwd(hipStream_t st, int M, int kh, int kw, const float* filters, float* ghat) {
    return rfft2_planes<FH, FW>(st, M, kh, kw, (size_t)kh * kw, true, filters,
                                reinterpret_cast<cpx*>(ghat));
}

template <int FH, int FW>
int spec_bwd(hipStream_t st, int M, int kh, int kw, int sh, int sw, const float* dghat,
             float* g, int acc, int conj_in) {
    const int rs = inv_rows<FH, FW>(kh);
    const size_t lds = linv_lds_bytes<FH, FW, kNT>(rs);
    set_lds(k_linv_filter<FH, FW>, lds);
    hipLaunchKernelGGL((k_linv_filter<FH, FW>), dim3(M, (kh + rs - 1) / rs), dim3(kNT), lds, st,
                       kh, kw, sh, sw, rs, reinterpret_cast<const cpx*>(dghat), g, acc, conj_in);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int corr(hipStream_t st, int B, int M, int hout, int wout, int ph, int pw, const float* xhat,
         const float* ghat, float* z, void* ws = nullptr, size_t ws_bytes = 0,
         float* stats = nullptr);

template <int FH, int FW>
int rfft2_two_pass(hipStream_t st, int nplanes, int hin, int win, size_t pstride, const float* x,
                   cpx* out, int nq = 1, size_t qstride = 0, const cpx* add = nullptr);

template <int FH, int FW>
int conv_fwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout, int ph, int pw,
             const float* x, int nq, const float* xhat_add, const float* ghat, float* z,
             float* xhat) {
    int rc = rfft2_two_pass<FH, FW>(st, B, hin, win, (size_t)hin * win, x,
                                    reinterpret_cast<cpx*>(xhat), nq, (size_t)B * hin * win,
                                    reinterpret_cast<const cpx*>(xhat_add));
    if (rc != NC_OK) return rc;
    return corr<FH, FW>(st, B, M, hout, wout, ph, pw, xhat, ghat, z);
}

// Bytes of the two-pass correlation's intermediate (B*M planes of hout x FW/2 cpx).
template <int FH, int FW>
size_t corr2_ws(int B, int M, int hout) {
    return (size_t)B * M * hout * LG<FH, FW>::NC * sizeof(cpx);
}

// Output rows per band of the row pass (the rows one workgroup finishes).
template <int FH, int FW>
constexpr int band_rows() {
    return 2 * (kNT / LG<FH, FW>::GW::G);
}

template <int FH, int FW>
int corr2(hipStream_t st, int B, int M, int hout, int wout, int ph, int pw, const float* xhat,
          const float* ghat, float* z, void* ws, float* stats) {
    using L = LG<FH, FW>;
    constexpr int CPW = kNT / L::GH::G, PPW = kNT / L::GW::G;
    cpx* T = reinterpret_cast<cpx*>(ws);
    hipLaunchKernelGGL((k_linv_cols<FH, FW, kSrcProduct>), dim3(L::NC / CPW, B * M), dim3(kNT), 0,
                       st, M, (size_t)0, hout, ph, reinterpret_cast<const cpx*>(xhat),
                       reinterpret_cast<const cpx*>(ghat), T);
    NC_CHECK_LAUNCH();
    const int npairs = (hout + 1) / 2;
    const dim3 grid((npairs + PPW - 1) / PPW, B * M);
    if (stats)
        hipLaunchKernelGGL((k_linv_rows<FH, FW, true>), grid, dim3(kNT), 0, st, hout, wout, pw,
                           1.0f / (float)(FH * FW), T, z, stats);
    else
        hipLaunchKernelGGL((k_linv_rows<FH, FW>), grid, dim3(kNT), 0, st, hout, wout, pw,
                           1.0f / (float)(FH * FW), T, z, nullptr);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

// Half-spectra of nplanes real planes (hin x win, pstride floats apart) by the two-pass
// transform, rows then columns in place in out.
template <int FH, int FW>
int rfft2_two_pass(hipStream_t st, int nplanes, int hin, int win, size_t pstride, const float* x,
                   cpx* out, int nq, size_t qstride, const cpx* add) {
    using L = LG<FH, FW>;
    constexpr int CPW = kNT / L::GH::G, PPW = kNT / L::GW::G;
    if (nplanes > 65535)  // the grid's y extent: one workgroup per plane segment instead
        return rfft2_planes<FH, FW>(st, nplanes, hin, win, pstride, false, x, out,
                                    add ? kPostAdd : kPostNone, SpecPost{add, 0, 0}, nq, qstride);
    const int npairs = (hin + 1) / 2;
    hipLaunchKernelGGL((k_lrfft_rows<FH, FW>), dim3((npairs + PPW - 1) / PPW, nplanes), dim3(kNT),
                       0, st, hin, win, pstride, nq, qstride, x, out);
    NC_CHECK_LAUNCH();
    hipLaunchKernelGGL((k_lrfft_cols<FH, FW>), dim3((L::SP + CPW - 1) / CPW, nplanes), dim3(kNT),
                       0, st, hin, add, out);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

// dx_b by the two-pass inverse: the sum of the nchunk partial spectra (nchunk, B, F), window
// rows / columns from the unshifted roll (FH - ph, FW - pw); T (B * hin * FW/2 cpx) is
// scratch.
template <int FH, int FW>
int dx_two_pass(hipStream_t st, int B, int nchunk, int hin, int win, int ph, int pw,
                const cpx* dxs, cpx* T, float* dx) {
    using L = LG<FH, FW>;
    constexpr int CPW = kNT / L::GH::G, PPW = kNT / L::GW::G;
    hipLaunchKernelGGL((k_linv_cols<FH, FW, kSrcChunks>), dim3(L::NC / CPW, B), dim3(kNT), 0, st,
                       nchunk, (size_t)B * L::F, hin, (FH - ph) & (FH - 1), dxs,
                       (const cpx*)nullptr, T);
    NC_CHECK_LAUNCH();
    const int npairs = (hin + 1) / 2;
    hipLaunchKernelGGL((k_linv_rows<FH, FW>), dim3((npairs + PPW - 1) / PPW, B), dim3(kNT), 0, st,
                       hin, win, (FW - pw) & (FW - 1), 1.0f / (float)(FH * FW), T, dx, nullptr);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int corr(hipStream_t st, int B, int M, int hout, int wout, int ph, int pw, const float* xhat,
         const float* ghat, float* z, void* ws, size_t ws_bytes, float* stats) {
    if (ws && ws_bytes >= corr2_ws<FH, FW>(B, M, hout) && (size_t)B * M <= 65535)
        return corr2<FH, FW>(st, B, M, hout, wout, ph, pw, xhat, ghat, z, ws, stats);
    if (stats) return NC_ERR_UNSUPPORTED;  // band statistics come from the two-pass row pass
    const int rs = inv_rows<FH, FW>(hout);
    const size_t lds = linv_lds_bytes<FH, FW, kNT>(rs);
    set_lds(k_linv_conv<FH, FW>, lds);
    hipLaunchKernelGGL((k_linv_conv<FH, FW>), dim3(B * M, (hout + rs - 1) / rs), dim3(kNT), lds,
                       st, M, hout, wout, ph, pw, rs, reinterpret_cast<const cpx*>(xhat),
                       reinterpret_cast<const cpx*>(ghat), z);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
size_t bwd_ws(int B, int M) {
    const int nchunk = (M + kRedMC - 1) / kRedMC;
    return ((size_t)B * M * FH * spec_pitch_ws<FH, FW>() + (size_t)nchunk * B * LG<FH, FW>::F) *
           sizeof(cpx);
}

template <int FH, int FW>
int seg_dx(hipStream_t st, int B, int nchunk, int hin, int win, int ph, int pw, const cpx* dxs,
           float* dx);

// epi: the cotangent planes are formed from the epilogue's inputs as the row pass reads them
// (gz unused), else read from gz.
template <int FH, int FW>
int conv_bwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout, int ph, int pw,
             const float* gz, const float* xhat, const float* ghat, int need_dx, float* dx,
             float* dghat, int accumulate, int conj_out, float* ssum, int sum_acc, int splits,
             void* ws, const nc_epi_gz* epi = nullptr) {
    using L = LG<FH, FW>;
    constexpr int SPP = spec_pitch_ws<FH, FW>();
    const int nchunk = (M + kRedMC - 1) / kRedMC;
    cpx* sp = reinterpret_cast<cpx*>(ws);
    cpx* part = sp + (size_t)B * M * FH * SPP;
    constexpr int CPW = kNT / L::GH::G, PPW = kNT / L::GW::G;
    const int npairs = (hout + 1) / 2;
    int pitch = SPP;
    if ((size_t)B * M > 65535) {  // beyond the passes' grid y extent: the segmented transform
        if (epi) return NC_ERR_UNSUPPORTED;
        int rc = rfft2_planes<FH, FW>(st, B * M, hout, wout, (size_t)hout * wout, false, gz, sp);
        if (rc != NC_OK) return rc;
        pitch = L::SP;
    } else if (epi) {
        auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
        const int vec = wout % 4 == 0 && al(epi->z) && al(epi->gy) && al(epi->w_eff) &&
                        al(epi->s_eff) && al(epi->b_roi);
        hipLaunchKernelGGL((k_lrfft_rows_epi<FH, FW, SPP>),
                           dim3((npairs + PPW - 1) / PPW, B * M), dim3(kNT), 0, st, M, hout,
                           wout, vec, *epi, sp);
    } else {
        hipLaunchKernelGGL((k_lrfft_rows<FH, FW, SPP>), dim3((npairs + PPW - 1) / PPW, B * M),
                           dim3(kNT), 0, st, hout, wout, (size_t)hout * wout, 1, (size_t)0, gz,
                           sp);
    }
    if (pitch == SPP) {
        NC_CHECK_LAUNCH();
        hipLaunchKernelGGL((k_lrfft_cols<FH, FW, SPP>), dim3((L::SP + CPW - 1) / CPW, B * M),
                           dim3(kNT), 0, st, hout, (const cpx*)nullptr, sp);
        NC_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL((k_lred<kRedMC>), dim3((FH * pitch + 255) / 256, nchunk, splits),
                       dim3(256), 0, st, B, M, L::F, L::SP, pitch, need_dx, sp,
                       reinterpret_cast<const cpx*>(xhat),
                       reinterpret_cast<const cpx*>(ghat), part, reinterpret_cast<cpx*>(dghat),
                       accumulate, conj_out, reinterpret_cast<cpx*>(ssum), sum_acc);
    NC_CHECK_LAUNCH();
    // the cotangent spectra are consumed: their region holds the dx passes' intermediate
    if (need_dx) return dx_two_pass<FH, FW>(st, B, nchunk, hin, win, ph, pw, part, sp, dx);
    return NC_OK;
}

// dx_b = the inverse of the sum of nchunk (nchunk, B, F) unpacked dx half-spectra, with the
// unshifted roll.
template <int FH, int FW, int NCH>
void seg_dx_launch(hipStream_t st, int B, int nchunk, int hin, int win, int ph, int pw,
                   const cpx* dxs, float* dx) {
    int rs = inv_rows<FH, FW>(hin);
    // few planes: more row segments (the column pass repeats per segment) to fill the CUs
    while (rs > 8 && (size_t)B * ((hin + rs - 1) / rs) < 256) rs = (rs + 1) / 2;
    const size_t lds = linv_lds_bytes<FH, FW, kNT>(rs);
    set_lds(k_linv_dx<FH, FW, NCH>, lds);
    hipLaunchKernelGGL((k_linv_dx<FH, FW, NCH>), dim3(B, (hin + rs - 1) / rs), dim3(kNT), lds, st,
                       B, nchunk, hin, win, ph, pw, rs, dxs, dx);
}

template <int FH, int FW>
int seg_dx(hipStream_t st, int B, int nchunk, int hin, int win, int ph, int pw, const cpx* dxs,
           float* dx) {
    if (nchunk == 1)
        seg_dx_launch<FH, FW, 1>(st, B, nchunk, hin, win, ph, pw, dxs, dx);
    else if (nchunk == 4)
        seg_dx_launch<FH, FW, 4>(st, B, nchunk, hin, win, ph, pw, dxs, dx);
    else
        seg_dx_launch<FH, FW, 0>(st, B, nchunk, hin, win, ph, pw, dxs, dx);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int hat_dx(hipStream_t st, int hin, int win, int ph, int pw, const cpx* dxs, float* dx) {
    return seg_dx<FH, FW>(st, 1, 1, hin, win, ph, pw, dxs, dx);
}

// The segmented transforms also serve the 64 x 64 grid's per-sample jobs (nc_seg_*).
#define NC_DISPATCH_SEG(FH_, FW_, CALL)                     \
    do {                                                    \
        if (FH_ == 64 && FW_ == 64) return CALL(64, 64);    \
        NC_DISPATCH_LARGE(FH_, FW_, CALL);                  \
    } while (0)

#define NC_DISPATCH_LARGE(FH_, FW_, CALL)                   \
    do {                                                    \
        if (FH_ == 64 && FW_ == 128) return CALL(64, 128);  \
        if (FH_ == 64 && FW_ == 256) return CALL(64, 256);  \
        if (FH_ == 128 && FW_ == 64) return CALL(128, 64);  \
        if (FH_ == 128 && FW_ == 128) return CALL(128, 128); \
        if (FH_ == 128 && FW_ == 256) return CALL(128, 256); \
        if (FH_ == 256 && FW_ == 64) return CALL(256, 64);  \
        if (FH_ == 256 && FW_ == 128) return CALL(256, 128); \
        if (FH_ == 256 && FW_ == 256) return CALL(256, 256); \
    } while (0)

}  // namespace

bool nc_large_grid(int fh, int fw) {
    auto ok = [](int f) { return f == 64 || f == 128 || f == 256; };
    return ok(fh) && ok(fw) && (fh > 64 || fw > 64);
}

int nc_large_filter_spectrum_fwd(hipStream_t st, int M, int kh, int kw, int fh, int fw,
                                 const float* filters, float* ghat) {
#define NC_CALL(A, Bv) spec_fwd<A, Bv>(st, M, kh, kw, filters, ghat)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_large_filter_spectrum_bwd(hipStream_t st, int M, int kh, int kw, int fh, int fw, int sh,
                                 int sw, const float* dghat, float* g, int acc, int conj_in) {
#define NC_CALL(A, Bv) spec_bwd<A, Bv>(st, M, kh, kw, sh, sw, dghat, g, acc, conj_in)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_large_fftconv_fwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout,
                         int ph, int pw, int fh, int fw, const float* x, int nq,
                         const float* xhat_add, const float* ghat, float* z, float* xhat) {
#define NC_CALL(A, Bv) \
    conv_fwd<A, Bv>(st, B, M, hin, win, hout, wout, ph, pw, x, nq, xhat_add, ghat, z, xhat)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

template <int FH, int FW>
int spectra(hipStream_t st, int n, const nc_spectrum_job* jobs) {
    if (n > kMaxLJobs) return NC_ERR_INVALID_ARGUMENT;
    LJobs J{};
    J.n = n;
    int hmax = 1;
    for (int q = 0; q < n; ++q) {
        const nc_spectrum_job& j = jobs[q];
        J.x[q] = j.x;
        J.out[q] = reinterpret_cast<cpx*>(j.xhat);
        J.post[q] = SpecPost{reinterpret_cast<const cpx*>(j.add), j.shift_h, j.shift_w};
        J.hin[q] = j.hin;
        J.win[q] = j.win;
        J.kind[q] = j.flip ? kLFlip : j.add ? kLAdd : (j.shift_h | j.shift_w) ? kLShift : kLPlain;
        J.start[q + 1] = J.start[q] + j.nplanes;
        hmax = std::max(hmax, j.hin);
    }
    // one column segmentation for all jobs: the LDS need grows with the live rows
    J.cs = fwd_cols<FH, FW>(hmax);
    const size_t lds = lfwd_lds_bytes<FH, FW, kNT>(hmax, J.cs);
    if (lds > kLdsMax) return NC_ERR_UNSUPPORTED;
    set_lds(k_lspectra<FH, FW>, lds);
    hipLaunchKernelGGL((k_lspectra<FH, FW>), dim3(J.start[n], LG<FH, FW>::NC / J.cs), dim3(kNT),
                       lds, st, J);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_large_plane_spectra(hipStream_t st, int fh, int fw, int n, const nc_spectrum_job* jobs) {
#define NC_CALL(A, Bv) spectra<A, Bv>(st, n, jobs)
    NC_DISPATCH_SEG(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_seg_rfft2(hipStream_t st, int fh, int fw, int nplanes, int hin, int win, int flip,
                 const float* x, void* xhat, const void* add, int sh, int sw, int nparts,
                 size_t qstride) {
    // large grids: the two-pass transform (rows, then columns in place)
    if (nc_large_grid(fh, fw) && !flip && !(sh | sw)) {
#define NC_CALL(A, Bv)                                                                        \
    rfft2_two_pass<A, Bv>(st, nplanes, hin, win, (size_t)hin * win, x,                       \
                          reinterpret_cast<cpx*>(xhat), nparts, qstride,                     \
                          reinterpret_cast<const cpx*>(add))
        NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    }
    const SpecPost post{reinterpret_cast<const cpx*>(add), sh, sw};
    const int kind = add ? kPostAdd : (sh | sw) ? kPostShift : kPostNone;
#define NC_CALL(A, Bv)                                                                    \
    rfft2_planes<A, Bv>(st, nplanes, hin, win, (size_t)hin * win, flip != 0, x,          \
                        reinterpret_cast<cpx*>(xhat), kind, post, nparts, qstride)
    NC_DISPATCH_SEG(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_seg_dx(hipStream_t st, int B, int nchunk, int hin, int win, int ph, int pw, int fh, int fw,
              const void* dxs, float* dx) {
#define NC_CALL(A, Bv) \
    seg_dx<A, Bv>(st, B, nchunk, hin, win, ph, pw, reinterpret_cast<const cpx*>(dxs), dx)
    NC_DISPATCH_SEG(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_large_correlate(hipStream_t st, int B, int M, int hout, int wout, int ph, int pw, int fh,
                       int fw, const float* xhat, const float* ghat, float* z, void* ws,
                       size_t ws_bytes, float* band_stats) {
#define NC_CALL(A, Bv) \
    corr<A, Bv>(st, B, M, hout, wout, ph, pw, xhat, ghat, z, ws, ws_bytes, band_stats)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_large_band_rows(int fh, int fw) {
#define NC_CALL(A, Bv) band_rows<A, Bv>()
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return 0;
}

size_t nc_large_band_stats_offset(int B, int M, int hout, int fh, int fw) {
#define NC_CALL(A, Bv) (corr2_ws<A, Bv>(B, M, hout) + 255) / 256 * 256
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return 0;
}

size_t nc_large_correlate_ws(int B, int M, int hout, int fh, int fw) {
    const int br = nc_large_band_rows(fh, fw);
    if (br == 0) return 0;
    const size_t bands = (size_t)(hout + br - 1) / br;
    return nc_large_band_stats_offset(B, M, hout, fh, fw) + 2 * (size_t)B * M * bands * 4;
}

int nc_large_plane_spectrum(hipStream_t st, int nplanes, int hin, int win, int fh, int fw, int sh,
                            int sw, const float* x, float* xhat) {
    const SpecPost post{nullptr, sh, sw};
#define NC_CALL(A, Bv)                                                                       \
    rfft2_planes<A, Bv>(st, nplanes, hin, win, (size_t)hin * win, false, x,                \
                        reinterpret_cast<cpx*>(xhat), kPostShift, post)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

size_t nc_large_fftconv_bwd_ws(int B, int M, int fh, int fw) {
#define NC_CALL(A, Bv) bwd_ws<A, Bv>(B, M)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return 0;
}

int nc_large_red_splits(int B, int M, int fh, int fw) {
    if (B <= 0 || M <= 0 || !nc_large_grid(fh, fw)) return 0;
    // sample slices that bring the reduction's grid to ~512 workgroups
    const int wgs = ((fh * (fw / 2 + 1) + 255) / 256) * ((M + kRedMC - 1) / kRedMC);
    const int want = std::max(1, std::min(B, (512 + wgs - 1) / wgs));
    const int bc = (B + want - 1) / want;
    return (B + bc - 1) / bc;
}

int nc_large_fftconv_bwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout,
                         int ph, int pw, int fh, int fw, const float* gz, const float* xhat,
                         const float* ghat, int need_dx, float* dx, float* dghat, int accumulate,
                         int conj_dghat, float* gz_hat_sum, int sum_accumulate, int parts,
                         void* ws) {
    const int splits = parts ? nc_large_red_splits(B, M, fh, fw) : 1;
#define NC_CALL(A, Bv)                                                                     \
    conv_bwd<A, Bv>(st, B, M, hin, win, hout, wout, ph, pw, gz, xhat, ghat, need_dx, dx, dghat, \
                    accumulate, conj_dghat, gz_hat_sum, sum_accumulate, splits, ws)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_large_fftconv_bwd_epi(hipStream_t st, int B, int M, int hin, int win, int hout,
                             int wout, int ph, int pw, int fh, int fw, const nc_epi_gz& gz,
                             const float* xhat, const float* ghat, int need_dx, float* dx,
                             float* dghat, int accumulate, int conj_dghat, float* gz_hat_sum,
                             int sum_accumulate, int parts, void* ws) {
    const int splits = parts ? nc_large_red_splits(B, M, fh, fw) : 1;
#define NC_CALL(A, Bv)                                                                        \
    conv_bwd<A, Bv>(st, B, M, hin, win, hout, wout, ph, pw, nullptr, xhat, ghat, need_dx, dx,  \
                    dghat, accumulate, conj_dghat, gz_hat_sum, sum_accumulate, splits, ws, &gz)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_large_hat_dx(hipStream_t st, int hin, int win, int ph, int pw, int fh, int fw,
                    const void* dxs, float* dx) {
#define NC_CALL(A, Bv) hat_dx<A, Bv>(st, hin, win, ph, pw, reinterpret_cast<const cpx*>(dxs), dx)
    NC_DISPATCH_LARGE(fh, fw, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

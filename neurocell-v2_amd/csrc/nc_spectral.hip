// Piece 2: Green's-function convolution as row-pruned overlap-save rfft2 correlation.
//
// Spectral grids of 16, 32 or 64 points per axis run wavefront-level transforms (nc_wave.h):
// one 64-lane wavefront owns PPW = 128 / FW planes, every 1D transform lives in one lane's
// registers and one LDS transposition separates the passes.  Spectra are (FH, FW/2+1)
// complex64 half-spectra in HBM; partial spectra use the packed (FH, FW/2) layout whose
// column 0 carries DC + i*Nyquist.
//
//   k_wrfft2<FLIP>        grid (planes/PPW)        half-spectra of real planes: the cell spectra
//                                                  xhat_b and (FLIP) ghat_m = rfft2(flip(G_m))
//   k_wconv_fwd           grid (B*M/PPW)           z_bm = irfft2(xhat_b * ghat_m), cropped window
//   k_wbwd_part           grid (M/PPW, B)          rfft2(gz_bm) once per plane, stored for the
//                                                  dG reduction; sum over the wave's directions
//                                                  of rfft2(gz_bm) * conj(ghat_m) (dx partials)
//   k_wbwd_dx_fin         grid (B/PPW)             fixed-order sum of those partials, irfft2 with
//                                                  the unshifted roll -> dx_b
//   k_wbwd_dg_red         grid (F/256, M, chunks)  fixed-order sums over sample chunks of the
//                                                  stored spectra times conj(xhat_b), unpacked
//   k_wbwd_dg_sum         grid (F/256, M)          fixed-order sum over the chunks -> dghat
//   k_filter_spectrum_bwd grid (M)                 dG_m = flip(crop(roll(irfft2(dghat_m))))
// No atomics anywhere: the M- and B-reductions are two-stage trees in the frequency domain.
#include <algorithm>
#include <cstdint>

#include "nc_large.h"

// nc_epilogue.hip: the port algebra over direction-group partial sums (2, G, B, P).
int nc_port_combine_launch(hipStream_t st, int B, int M, int P, int G, int final_act,
                           float neg_slope, const float* port_params, const float* part,
                           float* out, float* pre);
#include "nc_pair.h"
#include "nc_r8.h"
#include "nc_wave.h"

namespace {

// Plane pitch (cpx) of the stored cotangent half-spectra, padded to a multiple of 64.
template <int FH, int FW>
constexpr size_t spec_pitch() {
    return ((size_t)WGeo<FH, FW>::F + 63) / 64 * 64;
}

template <int FH, int FW>
struct Smem {
    using P = Plane<FH, FW>;
    cpx work[P::WORK];
    cpx scr[P::SCRN];
    cpx tw[NC_TW_N];
};

// Every workgroup-FFT kernel starts by copying the twiddle table into LDS.
#define NC_SPECTRAL_PROLOGUE(sm) \
    load_twiddles(sm.tw);        \
    __syncthreads()

// ----------------------------------------------------------------------------------------
// Filter spectrum backward (kernels_pallas.py:1558-1579)
// ----------------------------------------------------------------------------------------

template <int FH, int FW>
__global__ __launch_bounds__((Plane<FH, FW>::NT)) void k_filter_spectrum_bwd(
    int kh, int kw, int shift_h, int shift_w, const cpx* __restrict__ dghat,
    float* __restrict__ gfilt, int accumulate, int conj_in) {
    using P = Plane<FH, FW>;
    __shared__ Smem<FH, FW> sm;
    NC_SPECTRAL_PROLOGUE(sm);
    const int m = blockIdx.x;
    const cpx* d = dghat + (size_t)m * P::F;
    float* out = gfilt + (size_t)m * kh * kw;
    const int row0 = (FH - (shift_h % FH)) & (FH - 1);
    const int col0 = (FW - (shift_w % FW)) & (FW - 1);
    plane_irfft2<FH, FW>(
        [&](int a, int b) {
            const cpx v = d[a * P::SP + b];
            return conj_in ? cconj(v) : v;
        },
        row0, kh, col0, kw, 1.0f / (float)(FH * FW),
        [&](int i, int j, float v) {
            float* o = out + (kh - 1 - i) * kw + (kw - 1 - j);
            *o = accumulate ? *o + v : v;
        },
        sm.work, sm.scr, sm.tw);
}

// The filter gradients and the border patch's gradient in one launch: workgroups m < M as
// k_filter_spectrum_bwd; workgroup M inverts the patch's cotangent spectrum pspec (unpacked,
// k_hat_red's sum over m of S_m conj(ghat_m): the one-sample correlation backward of
// kernels_pallas.py:1794-1812), rolled by (pshift_h, pshift_w) and cropped to (hp, wp).
template <int FH, int FW>
__global__ __launch_bounds__((Plane<FH, FW>::NT)) void k_filter_patch_bwd(
    int M, int kh, int kw, int shift_h, int shift_w, const cpx* __restrict__ dghat,
    float* __restrict__ gfilt, int accumulate, int conj_in, int hp, int wp, int pshift_h,
    int pshift_w, const cpx* __restrict__ pspec, float* __restrict__ gpatch) {
    using P = Plane<FH, FW>;
    __shared__ Smem<FH, FW> sm;
    NC_SPECTRAL_PROLOGUE(sm);
    const int m = blockIdx.x;
    const float scale = 1.0f / (float)(FH * FW);
    if (m < M) {
        const cpx* d = dghat + (size_t)m * P::F;
        float* out = gfilt + (size_t)m * kh * kw;
        plane_irfft2<FH, FW>(
            [&](int a, int b) {
                const cpx v = d[a * P::SP + b];
                return conj_in ? cconj(v) : v;
            },
            (FH - (shift_h % FH)) & (FH - 1), kh, (FW - (shift_w % FW)) & (FW - 1), kw, scale,
            [&](int i, int j, float v) {
                float* o = out + (kh - 1 - i) * kw + (kw - 1 - j);
                *o = accumulate ? *o + v : v;
            },
            sm.work, sm.scr, sm.tw);
    } else {
        plane_irfft2<FH, FW>(
            [&](int a, int b) { return pspec[a * P::SP + b]; },
            (FH - (pshift_h % FH)) & (FH - 1), hp, (FW - (pshift_w % FW)) & (FW - 1), wp, scale,
            [&](int i, int j, float v) { gpatch[i * wp + j] = v; }, sm.work, sm.scr, sm.tw);
    }
}

// ----------------------------------------------------------------------------------------
// Wavefront kernels (one 64-lane wavefront per workgroup)
// ----------------------------------------------------------------------------------------

// Half-spectra of nplanes real (hin x win) planes stored back to back in x (FLIP: the plane
// is read flipped in both axes, which turns the correlation filter into a convolution
// kernel, kernels_greens.py:240-259).  out: (nplanes, FH, FW/2+1).
template <int FH, int FW, bool FLIP, int POST, int NP>
__global__ __launch_bounds__(64) void k_wrfft2(int nplanes, int hin, int win, int s_off, int vec,
                                               const float* __restrict__ x,
                                               cpx* __restrict__ out, SpecPost post,
                                               size_t qstride, int nq) {
    using W = WGeo<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    cpx* T = reinterpret_cast<cpx*>(lds);
    float* S = lds + s_off;
    const int lane = threadIdx.x;
    const int g0 = blockIdx.x * W::PPW;
    const int np = min(W::PPW, nplanes - g0);
    istage<FW, W::PPW, FLIP, NP>(x + (size_t)g0 * hin * win, (size_t)hin * win, np, hin, win,
                                 vec != 0, S, qstride, nq);
    __syncthreads();
    wrow_fwd<FH, FW>(S, hin, T);
    __syncthreads();
    cpx v[FH];
    wcol_fwd<FH, FW>(T, hin, v);
    const int ps = lane / W::NC, kc = lane % W::NC;
    if (ps >= np) return;
    cpx* o = out + (size_t)(g0 + ps) * W::F + kc;
    if (kc == 0) {
#pragma unroll
        for (int kh = 0; kh < FH; ++kh) {
            const cpx c = v[kh], d = cconj(v[(FH - kh) & (FH - 1)]);
            o[kh * W::SP] = spec_post<POST, FH, FW>(cscale(cadd(c, d), 0.5f), kh, 0, post);
            o[kh * W::SP + FW / 2] =
                spec_post<POST, FH, FW>(cmul_negi(cscale(csub(c, d), 0.5f)), kh, FW / 2, post);
        }
    } else {
#pragma unroll
        for (int kh = 0; kh < FH; ++kh) o[kh * W::SP] = spec_post<POST, FH, FW>(v[kh], kh, kc, post);
    }
}

// Forward correlation (kernels_pallas.py:1779-1791; kernels_greens.py:316-343): plane
// g = b*M + m of z (B, M, hout, wout) is irfft2(xhat_b * ghat_m) read from row ph, column pw.
template <int FH, int FW>
__global__ __launch_bounds__(64) void k_wconv_fwd(int nplanes, int M, int hout, int wout, int ph,
                                                  int pw, int o_off, int nq_off, int vec,
                                                  const cpx* __restrict__ xhat,
                                                  const cpx* __restrict__ ghat,
                                                  float* __restrict__ z) {
    using W = WGeo<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    cpx* T = reinterpret_cast<cpx*>(lds);
    float* O = lds + o_off;
    cpx* NQ = reinterpret_cast<cpx*>(lds) + nq_off;
    const int lane = threadIdx.x, ps = lane / W::NC, kc = lane % W::NC;
    const int g0 = blockIdx.x * W::PPW;
    const int np = min(W::PPW, nplanes - g0);
    const int g = g0 + min(ps, np - 1);
    const int b = g / M, m = g - b * M;
    const cpx* X = xhat + (size_t)b * W::F;
    const cpx* G = ghat + (size_t)m * W::F;
    cpx v[FH];
#pragma unroll
    for (int kh = 0; kh < FH; ++kh) v[kh] = cmul(X[kh * W::SP + kc], G[kh * W::SP + kc]);
    // Nyquist-column products, spread over the lanes, for the packed column
    for (int kh = kc; kh < FH; kh += W::NC)
        NQ[ps * FH + kh] = cmul(X[kh * W::SP + FW / 2], G[kh * W::SP + FW / 2]);
    __syncthreads();
    if (kc == 0) {
#pragma unroll
        for (int kh = 0; kh < FH; ++kh) v[kh] = cadd(v[kh], cmul_i(NQ[ps * FH + kh]));
    }
    wcol_inv<FH, FW>(v, ph, hout, T);
    __syncthreads();
    wrow_inv<FH, FW>(T, pw, hout, 1.0f / (float)(FH * FW), O);
    __syncthreads();
    ostage_copy<FW>(O, np, hout, wout, z + (size_t)g0 * hout * wout);
}

// Backward first stage (kernels_pallas.py:1794-1821), in the packed layout.  Wavefront
// (mg, b) transforms the gz planes (b, m = mg*PPW + ps) once; it stores each plane's
// half-spectrum in spec (M, B, pitch) for the dG reduction (k_wbwd_dg_red) and, when need_dx, writes
// part[b][mg] = sum over its planes of rfft2(gz_bm) * conj(ghat_m) for the dx chain.  Planes
// past M are staged as zeros and contribute nothing.
template <int FH, int FW>
__global__ __launch_bounds__(64) void k_wbwd_part(int B, int M, int hout, int wout, int s_off,
                                                  int nq_off, int vec, int need_dx,
                                                  const float* __restrict__ gz,
                                                  const cpx* __restrict__ ghat,
                                                  cpx* __restrict__ part,
                                                  cpx* __restrict__ spec) {
    using W = WGeo<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    cpx* T = reinterpret_cast<cpx*>(lds);
    float* S = lds + s_off;
    cpx* NQ = reinterpret_cast<cpx*>(lds) + nq_off;
    const int lane = threadIdx.x, ps = lane / W::NC, kc = lane % W::NC;
    const size_t n = (size_t)hout * wout;
    const int b0 = blockIdx.y;
    const int m0 = blockIdx.x * W::PPW;
    const int np = min(W::PPW, M - m0);
    istage<FW, W::PPW, false>(gz + ((size_t)b0 * M + m0) * n, n, np, hout, wout, vec != 0, S);
    const int q = min(ps, np - 1);
    const cpx* R = ghat + (size_t)(m0 + q) * W::F;
    cpx r[FH];  // the reference column, loaded while the transform runs
    if (need_dx) {
#pragma unroll
        for (int kh = 0; kh < FH; ++kh) r[kh] = R[kh * W::SP + kc];
        stage_nyquist<FH, FW>([&](int p) { return ghat + (size_t)(m0 + min(p, np - 1)) * W::F; },
                              NQ);
    }
    __syncthreads();
    wrow_fwd<FH, FW>(S, hout, T);
    __syncthreads();
    cpx v[FH];
    wcol_fwd<FH, FW>(T, hout, v);
    if (ps < np) {
        // half-spectrum of the plane: the lane of packed column 0 splits DC + i*Nyquist with
        // its row mirrors (all in its registers) into the DC and Nyquist columns
        cpx* o = spec + ((size_t)(m0 + ps) * B + b0) * spec_pitch<FH, FW>() + kc;
        if (kc != 0) {
#pragma unroll
            for (int kh = 0; kh < FH; ++kh) o[kh * W::SP] = v[kh];
        } else {
#pragma unroll
            for (int kh = 0; kh < FH; ++kh) {
                const cpx c = v[kh], d = cconj(v[(FH - kh) & (FH - 1)]);
                o[kh * W::SP] = cscale(cadd(c, d), 0.5f);
                o[kh * W::SP + FW / 2] = cmul_negi(cscale(csub(c, d), 0.5f));
            }
        }
    }
    if (!need_dx) return;  // uniform over the launch
    packed_mulc<FH>(v, r, kc, [&](int kh) { return NQ[ps * FH + kh]; });
    // sum over the wavefront's planes, half a spectrum at a time, through T
    constexpr int HH = FH / 2;
    cpx* red = T;
    cpx* dst = part + ((size_t)b0 * gridDim.x + blockIdx.x) * W::PF;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        __syncthreads();
#pragma unroll
        for (int k = 0; k < HH; ++k) red[(ps * HH + k) * W::NC + kc] = v[h * HH + k];
        __syncthreads();
#pragma unroll
        for (int e0 = 0; e0 < HH * W::NC; e0 += 64) {
            const int e = e0 + lane;
            cpx acc = red[e];
#pragma unroll
            for (int p = 1; p < W::PPW; ++p) acc = cadd(acc, red[p * HH * W::NC + e]);
            dst[h * HH * W::NC + e] = acc;
        }
    }
}

// Fixed-order sum of n complex values p[0], p[stride], ... with eight independent chains
// (combined in a fixed tree), so each thread keeps eight loads in flight.
NC_DEV cpx sum_strided(const cpx* __restrict__ p, int n, size_t stride) {
    cpx a[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) a[u] = cmk(0.f, 0.f);
    int j = 0;
    for (; j + 8 <= n; j += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) a[u] = cadd(a[u], p[(size_t)(j + u) * stride]);
    }
    for (; j < n; ++j) a[0] = cadd(a[0], p[(size_t)j * stride]);
    return cadd(cadd(cadd(a[0], a[1]), cadd(a[2], a[3])), cadd(cadd(a[4], a[5]), cadd(a[6], a[7])));
}

// out[i][e] = sum over j < nj of in[i * istride + j * jstride + e], e < len (grid (len/256, ni)).
__global__ void k_psum(int nj, int len, size_t istride, size_t jstride, const cpx* __restrict__ in,
                       cpx* __restrict__ out) {
    const int i = blockIdx.y;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= len) return;
    out[(size_t)i * len + e] = sum_strided(in + (size_t)i * istride + e, nj, jstride);
}

// dx, second stage: the inverse of the summed packed spectrum of sample b with the unshifted
// roll (kernels_pallas.py:1798-1812): rows from (FH - ph) mod FH, columns from (FW - pw) mod FW,
// hin x win kept.
template <int FH, int FW>
__global__ __launch_bounds__(64) void k_wbwd_dx_fin(int B, int hin, int win, int ph, int pw,
                                                    int o_off, int vec,
                                                    const cpx* __restrict__ sum,
                                                    float* __restrict__ dx) {
    using W = WGeo<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    cpx* T = reinterpret_cast<cpx*>(lds);
    float* O = lds + o_off;
    const int lane = threadIdx.x, ps = lane / W::NC, kc = lane % W::NC;
    const int b0 = blockIdx.x * W::PPW;
    const int np = min(W::PPW, B - b0);
    const cpx* src = sum + (size_t)(b0 + min(ps, np - 1)) * W::PF + kc;
    cpx v[FH];
#pragma unroll
    for (int kh = 0; kh < FH; ++kh) v[kh] = src[kh * W::NC];
    wcol_inv<FH, FW>(v, (FH - ph) & (FH - 1), hin, T);
    __syncthreads();
    wrow_inv<FH, FW>(T, (FW - pw) & (FW - 1), hin, 1.0f / (float)(FH * FW), O);
    __syncthreads();
    ostage_copy<FW>(O, np, hin, win, dx + (size_t)b0 * hin * win);
}

constexpr int kDgBatch = 16;  // samples whose loads a dG-reduction thread keeps in flight

// dG reduction (kernels_pallas.py:1818-1820), first stage: over the samples of chunk
// c = blockIdx.z, in increasing b, of rfft2(gz_bm) * conj(xhat_b), bin by bin, from the stored
// half-spectra spec (M, B, pitch).  With one chunk the result goes to dghat directly
// (conj_out: conjugate convention, accumulate: add); otherwise to part (chunks, M, F) for
// k_wbwd_dg_sum.  With ssum the plain sums over b of rfft2(gz_bm) are formed alongside (the
// spectra of sum_b gz_bm, by linearity), into ssum (M, F) or the partial rows
// part[chunks + c] (added to ssum when sum_acc).
// parts_mode: dghat and ssum are row stacks (chunks, M, F); chunk c's sums are written to (or
// added to, accumulate / sum_acc) their row c, conjugated per row when conj_out, and no
// chunk sum runs - the consumer adds the rows (nc_filter_spectrum_bwd_parts, ..._hat_parts).
template <int FH, int FW>
__global__ __launch_bounds__(256) void k_wbwd_dg_red(int B, int M, int bper,
                                                     const cpx* __restrict__ spec,
                                                     const cpx* __restrict__ xhat,
                                                     cpx* __restrict__ part,
                                                     cpx* __restrict__ dghat, int accumulate,
                                                     int conj_out, cpx* __restrict__ ssum,
                                                     int sum_acc, int parts_mode) {
    using W = WGeo<FH, FW>;
    constexpr size_t SPP = spec_pitch<FH, FW>();
    const int m = blockIdx.y, c = blockIdx.z;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= W::F) return;
    const int b0 = c * bper, b1 = min(B, b0 + bper);
    const cpx* S = spec + (size_t)m * B * SPP + e;
    const cpx* X = xhat + e;
    cpx acc = cmk(0.f, 0.f), sacc = cmk(0.f, 0.f);
    for (int bb = b0; bb < b1; bb += kDgBatch) {
        // the batch's loads are issued together (clamped), then added in increasing b
        cpx u[kDgBatch], xv[kDgBatch];
#pragma unroll
        for (int j = 0; j < kDgBatch; ++j) {
            const int b = min(bb + j, b1 - 1);
            u[j] = S[(size_t)b * SPP];
            xv[j] = X[(size_t)b * W::F];
        }
#pragma unroll
        for (int j = 0; j < kDgBatch; ++j) {
            if (bb + j < b1) {
                acc = cadd(acc, cmulc(u[j], xv[j]));
                sacc = cadd(sacc, u[j]);
            }
        }
    }
    if (gridDim.z == 1 || parts_mode) {
        const size_t row = parts_mode ? (size_t)c * M : 0;
        if (conj_out) acc = cconj(acc);
        cpx* o = dghat + (row + m) * W::F + e;
        *o = accumulate ? cadd(*o, acc) : acc;
        if (ssum) {
            cpx* so = ssum + (row + m) * W::F + e;
            *so = sum_acc ? cadd(*so, sacc) : sacc;
        }
    } else {
        part[((size_t)c * M + m) * W::F + e] = acc;
        if (ssum) part[((size_t)(gridDim.z + c) * M + m) * W::F + e] = sacc;
    }
}

// dG reduction, second stage: dghat[m] (+)= sum over the chunks in order (grid (F/256, M, 1));
// with a second grid layer (blockIdx.z == 1) also ssum[m] (+)= the chunks' plain sums.
__global__ __launch_bounds__(256) void k_wbwd_dg_sum(int nchunk, int M, int F,
                                                     const cpx* __restrict__ part,
                                                     cpx* __restrict__ dghat, int accumulate,
                                                     int conj_out, cpx* __restrict__ ssum,
                                                     int sum_acc) {
    const int m = blockIdx.y;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= F) return;
    if (blockIdx.z == 0) {
        cpx v = sum_strided(part + (size_t)m * F + e, nchunk, (size_t)M * F);
        if (conj_out) v = cconj(v);
        cpx* o = dghat + (size_t)m * F + e;
        *o = accumulate ? cadd(*o, v) : v;
    } else {
        const cpx v = sum_strided(part + ((size_t)nchunk * M + m) * F + e, nchunk, (size_t)M * F);
        cpx* o = ssum + (size_t)m * F + e;
        *o = sum_acc ? cadd(*o, v) : v;
    }
}

// Backward of a one-sample correlation from its cotangent half-spectra S (M, F), the
// spectra of gz (kernels_pallas.py:1794-1821 at B = 1): dghat[m] (+)= S_m * conj(xhat)
// (conjugated when conj_out; skipped without dghat) and the dx spectrum sum over m, in
// increasing order, of S_m * conj(ghat_m), into dxs: unpacked (FH, FW/2 + 1) or, with packed,
// the (FH, FW/2) layout whose column 0 holds DC + i*Nyquist.  Thread = packed bin (kh, kc);
// kc == 0 also carries column FW/2.
__global__ __launch_bounds__(256) void k_hat_red(int M, int FH, int FWh, int packed,
                                                 const cpx* __restrict__ S,
                                                 const cpx* __restrict__ xhat,
                                                 const cpx* __restrict__ ghat,
                                                 cpx* __restrict__ dxs, cpx* __restrict__ dghat,
                                                 int accumulate, int conj_out) {
    constexpr int MC = 8;
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= FH * FWh) return;
    const int kh = p / FWh, kc = p - kh * FWh;
    const int F = FH * (FWh + 1);
    const int e0 = kh * (FWh + 1) + kc, e1 = kh * (FWh + 1) + FWh;
    const bool two = kc == 0;
    const cpx X0 = dghat ? xhat[e0] : cmk(0.f, 0.f);
    const cpx X1 = dghat ? xhat[e1] : cmk(0.f, 0.f);
    cpx d0 = cmk(0.f, 0.f), d1 = cmk(0.f, 0.f);
    for (int m0 = 0; m0 < M; m0 += MC) {
        cpx s0[MC], s1[MC], g0[MC], g1[MC];
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            const size_t o = (size_t)min(m0 + q, M - 1) * F;
            s0[q] = S[o + e0];
            s1[q] = S[o + e1];
            g0[q] = ghat[o + e0];
            g1[q] = ghat[o + e1];
        }
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            if (m0 + q >= M) break;
            d0 = cadd(d0, cmulc(s0[q], g0[q]));
            d1 = cadd(d1, cmulc(s1[q], g1[q]));
            if (dghat) {
                const size_t o = (size_t)(m0 + q) * F;
                cpx v = cmulc(s0[q], X0);
                if (conj_out) v = cconj(v);
                dghat[o + e0] = accumulate ? cadd(dghat[o + e0], v) : v;
                if (two) {
                    cpx w = cmulc(s1[q], X1);
                    if (conj_out) w = cconj(w);
                    dghat[o + e1] = accumulate ? cadd(dghat[o + e1], w) : w;
                }
            }
        }
    }
    if (packed) {
        dxs[p] = two ? cadd(d0, cmul_i(d1)) : d0;
    } else {
        dxs[e0] = d0;
        if (two) dxs[e1] = d1;
    }
}

// ----------------------------------------------------------------------------------------
// Lane-pair kernels for 64-wide grids (nc_pair.h): one plane per wavefront
// ----------------------------------------------------------------------------------------

template <int FH, int FW>
constexpr bool pair_grid() {
    return FW == 64 && (FH == 32 || FH == 64);
}

// On the 64 x 64 grid the per-sample transforms (cell spectra, dx inverses, the few-plane
// filter and border spectra) run as workgroup-per-plane segmented transforms: with one
// wavefront per plane a B-plane job leaves most of the chip idle and its time is one
// wavefront's latency; the B*M-plane correlation and cotangent spectra stay lane-pair.
template <int FH, int FW>
constexpr bool seg_grid() {
    return FH == 64 && FW == 64;
}

// LDS of a lane-pair plane: T (forward: `rows` + 2 rows; inverse: all fh rows) of pitch cpx,
// sharing its space with the real-valued input or output staging, then the Nyquist staging
// (fh cpx).
struct PLds {
    size_t bytes;
    int nq;  // cpx offset of the Nyquist staging
    PLds(int rows, int pitch, int fw, int fh, bool inverse, bool window = false) {
        // the inverse's T: all fh rows (only the window's `rows` with pcol_inv_rows) and the
        // gap between its two row halves
        const int trows = inverse ? (window ? rows : fh) : rows + 2;
        const size_t t = ((size_t)trows * pitch + (inverse ? kPairGap : 0)) * sizeof(cpx);
        const size_t o = (size_t)(rows + 1) * (fw + 1) * sizeof(float);
        const size_t main = (std::max(t, o) + 15) / 16 * 16;
        nq = (int)(main / sizeof(cpx));
        bytes = main + (size_t)fh * sizeof(cpx);
    }
};

// Half-spectrum of one real (hin x win) plane src into o (FLIP: read rotated by 180 degrees),
// each bin passed through spec_post<POST>; the calling wavefront owns the plane.  kPostAdd
// loads the lane's added bins while the column transform runs, so no store waits on a load.
template <int FH, int FW, bool FLIP, int POST, int NP = 1>
NC_DEV void prfft2_plane(const float* __restrict__ src, int hin, int win, int vec, float* lds,
                         cpx* __restrict__ o, const SpecPost& post, size_t qstride = 0,
                         int nq = 1) {
    using P = PGeo<FH, FW>;
    constexpr int NA = POST == kPostAdd ? P::HH : 1;
    cpx* T = reinterpret_cast<cpx*>(lds);
    istage<FW, 1, FLIP, NP>(src, (size_t)hin * win, 1, hin, win, vec != 0, lds, qstride, nq);
    __syncthreads();
    prow_fwd<FH, FW>(lds, hin, T);
    __syncthreads();
    cpx av[NA], an[NA];  // bins (t*HH + k, kc) and, for column 0's split, (t*HH + k, FW/2)
    if constexpr (POST == kPostAdd) {
        const int lane = threadIdx.x & 63, kc = lane >> 1, t = lane & 1;
        const cpx* a = post.add + (size_t)t * P::HH * P::SP;
#pragma unroll
        for (int k = 0; k < P::HH; ++k) {
            av[k] = a[k * P::SP + kc];
            an[k] = a[k * P::SP + FW / 2];
        }
    }
    cpx v[P::HH];
    pcol_fwd<FH, FW>(T, hin, v);
    pstore_half<FH, FW>(v, [&](int k, int kh, int kw, cpx val) {
        if constexpr (POST == kPostAdd) val = cadd(val, kw == FW / 2 ? an[k] : av[k]);
        if constexpr (POST == kPostShift) val = spec_post<POST, FH, FW>(val, kh, kw, post);
        o[kh * P::SP + kw] = val;
    });
}

// Half-spectra of real (hin x win) planes (FLIP: read rotated by 180 degrees, the filter
// spectra of kernels_greens.py:240-259), post-processed by spec_post<POST>; one wavefront per
// plane.
template <int FH, int FW, bool FLIP, int POST, int NP>
__global__ __launch_bounds__(64) void k_prfft2(int hin, int win, int vec,
                                               const float* __restrict__ x,
                                               cpx* __restrict__ out, SpecPost post,
                                               size_t qstride, int nq) {
    HIP_DYNAMIC_SHARED(float, lds)
    prfft2_plane<FH, FW, FLIP, POST, NP>(x + (size_t)blockIdx.x * hin * win, hin, win, vec, lds,
                                         out + (size_t)blockIdx.x * PGeo<FH, FW>::F, post,
                                         qstride, nq);
}

// Backward, first stage (kernels_pallas.py:1794-1821): the half-spectrum of every cotangent
// plane gz_bm (g = b*M + m) into spec (M, B, pitch), one wavefront per plane.
template <int FH, int FW>
__global__ __launch_bounds__(64) void k_pspec(int B, int M, int hout, int wout, int vec,
                                              const float* __restrict__ gz,
                                              cpx* __restrict__ spec) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int g = blockIdx.x, b = g / M, m = g - b * M;
    prfft2_plane<FH, FW, false, kPostNone>(gz + (size_t)g * hout * wout, hout, wout, vec, lds,
                                           spec + ((size_t)m * B + b) * spec_pitch<FH, FW>(),
                                           SpecPost{});
}

// Stages one (hin x win) real plane at the origin of the 64 x 64 grid into the radix-8 input
// staging S (hin rows of r8::kSP floats, columns win..63 zero), as r8::fwd_plane expects it.
// The plane's n <= 4096 floats are read lane by lane (element f = tid + 256 u), all loads
// issued together; with NP != 1 each element is the sum of the partial planes qstride floats
// apart, in increasing order (NP == 0: nq of them).  Consecutive lanes write consecutive
// columns, so the stores meet no bank conflicts.
template <int NP>
NC_DEV void r8_stage_plane(const float* __restrict__ src, int hin, int win, size_t qstride,
                           int nq, float* S) {
    const int tid = threadIdx.x, n = hin * win;
    constexpr int U = 16;
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int f = tid + u * r8::kNT;
        float a = 0.f;
        if (f < n) {
            a = src[f];
            if constexpr (NP > 1) {
#pragma unroll
                for (int q = 1; q < NP; ++q) a += src[q * qstride + f];
            } else if constexpr (NP == 0) {
                for (int q = 1; q < nq; ++q) a += src[q * qstride + f];
            }
        }
        v[u] = a;
    }
    for (int e = tid; e < hin * (64 - win); e += r8::kNT) {
        const int r = e / (64 - win);
        S[r * r8::kSP + win + (e - r * (64 - win))] = 0.f;
    }
    const unsigned inv = ((1u << 20) + win - 1) / win;  // exact floor(f / win), f < 4096
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int f = tid + u * r8::kNT;
        if (f < n) {
            const int r = (int)(((unsigned)f * inv) >> 20);
            S[r * r8::kSP + (f - r * win)] = v[u];
        }
    }
}

// Backward, first stage on the 64 x 64 grid: the half-spectrum of every cotangent plane
// gz_bm (g = b*M + m) into spec (M, B, pitch), one 256-thread workgroup per plane (8-lane
// 64-point transforms, nc_r8.h): the plane is staged in LDS with coalesced loads, transformed,
// and its half-spectrum stored with 16-byte stores.
__global__ __launch_bounds__(r8::kNT) void k_r8spec(int B, int M, int hout, int wout,
                                                    const float* __restrict__ gz,
                                                    cpx* __restrict__ spec) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int g = blockIdx.x, b = g / M, m = g - b * M, tid = threadIdx.x;
    const r8::Tw tw = r8::twiddles(tid & 7);
    r8_stage_plane<1>(gz + (size_t)g * hout * wout, hout, wout, 0, 1, lds + 2 * r8::kExCpx);
    r8::fwd_plane(lds, hout, tw);
    const cpx* O = reinterpret_cast<const cpx*>(lds + 2 * r8::kExCpx);
    cpx* dst = spec + ((size_t)m * B + b) * spec_pitch<64, 64>();
#pragma unroll
    for (int u = 0; u < (r8::kF + r8::kNT - 1) / r8::kNT; ++u) {
        const int e = tid + u * r8::kNT;
        if (e < r8::kF) {
            const int kh = e / 33, kw = e - 33 * kh;
            dst[e] = O[kh * r8::kOP + kw];
        }
    }
}

// Half-spectra (64, 33) of real (hin x win) planes on the 64 x 64 grid, one 256-thread
// workgroup per plane (the cell spectra of a propagation step: each plane the sum of the
// previous step's direction-group partial outputs, kernels_pallas.py:1779-1791), each bin
// through spec_post<POST> (kPostNone or kPostAdd: plus the shared border-patch spectrum).
template <int POST, int NP>
__global__ __launch_bounds__(r8::kNT) void k_r8rfft2(int hin, int win, size_t qstride, int nq,
                                                     const float* __restrict__ x,
                                                     cpx* __restrict__ out, SpecPost post) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int g = blockIdx.x, tid = threadIdx.x;
    const r8::Tw tw = r8::twiddles(tid & 7);
    r8_stage_plane<NP>(x + (size_t)g * hin * win, hin, win, qstride, nq, lds + 2 * r8::kExCpx);
    r8::fwd_plane(lds, hin, tw);
    const cpx* O = reinterpret_cast<const cpx*>(lds + 2 * r8::kExCpx);
    cpx* dst = out + (size_t)g * r8::kF;
#pragma unroll
    for (int u = 0; u < (r8::kF + r8::kNT - 1) / r8::kNT; ++u) {
        const int e = tid + u * r8::kNT;
        if (e < r8::kF) {
            const int kh = e / 33, kw = e - 33 * kh;
            dst[e] = spec_post<POST, 64, 64>(O[kh * r8::kOP + kw], kh, kw, post);
        }
    }
}

// Backward, both frequency-domain reductions in one pass over the stored cotangent spectra
// spec (M, B, pitch) (kernels_pallas.py:1794-1821).  Workgroup = 64 bins x 4 waves, wave g
// owning the directions [g*MG, (g+1)*MG); blockIdx.y = sample chunk c:
//   dxs[b][e]      = sum over m of spec_mb * conj(ghat_m): each wave sums its directions
//                    (increasing m), the four wave sums are added in order through LDS
//   dgrow[c][m][e] (+)= sum over the chunk's samples, increasing, of spec_mb * conj(xhat_b)
//                    (conjugated when conj_out)
//   srow[c][m][e]  (+)= sum over the chunk's samples of spec_mb (with srow)
// Each spectrum value is read once for both sums; kPBB samples' loads are in flight together.
constexpr int kPBB = 4;

template <int FH, int FW, int MG>
__global__ __launch_bounds__(256) void k_pbwd_red(int B, int M, int bper, int need_dx,
                                                  const cpx* __restrict__ spec,
                                                  const cpx* __restrict__ xhat,
                                                  const cpx* __restrict__ ghat,
                                                  cpx* __restrict__ dxs, cpx* __restrict__ dgrow,
                                                  int accumulate, int conj_out,
                                                  cpx* __restrict__ srow, int sum_acc) {
    using P = PGeo<FH, FW>;
    constexpr size_t SPP = spec_pitch<FH, FW>();
    __shared__ cpx red[4][kPBB][64];
    const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
    const int e0 = blockIdx.x * 64 + lane, e = min(e0, P::F - 1);
    const int c = blockIdx.y;
    const int m0 = g * MG, nm = max(0, min(MG, M - m0));
    const int b0 = c * bper, b1 = min(B, b0 + bper);
    cpx G[MG], dg[MG], sg[MG];
#pragma unroll
    for (int q = 0; q < MG; ++q) {
        G[q] = ghat[(size_t)min(m0 + q, M - 1) * P::F + e];
        dg[q] = sg[q] = cmk(0.f, 0.f);
    }
    for (int bb = b0; bb < b1; bb += kPBB) {
        cpx u[kPBB][MG], xv[kPBB];
#pragma unroll
        for (int j = 0; j < kPBB; ++j) {
            const int b = min(bb + j, b1 - 1);
            xv[j] = xhat[(size_t)b * P::F + e];
#pragma unroll
            for (int q = 0; q < MG; ++q)
                u[j][q] = spec[((size_t)min(m0 + q, M - 1) * B + b) * SPP + e];
        }
#pragma unroll
        for (int j = 0; j < kPBB; ++j) {
            cpx d = cmk(0.f, 0.f);
            const bool on = bb + j < b1;
#pragma unroll
            for (int q = 0; q < MG; ++q) {
                if (q < nm && on) {
                    d = cadd(d, cmulc(u[j][q], G[q]));
                    dg[q] = cadd(dg[q], cmulc(u[j][q], xv[j]));
                    sg[q] = cadd(sg[q], u[j][q]);
                }
            }
            red[g][j][lane] = d;
        }
        __syncthreads();
        if (need_dx) {  // wave g finishes samples j = g, g + 4, ...: the four wave sums in order
            for (int j = g; j < kPBB && bb + j < b1; j += 4) {
                const cpx v = cadd(cadd(cadd(red[0][j][lane], red[1][j][lane]), red[2][j][lane]),
                                   red[3][j][lane]);
                if (e0 < P::F) dxs[(size_t)(bb + j) * P::F + e0] = v;
            }
        }
        __syncthreads();
    }
    if (e0 >= P::F) return;
#pragma unroll
    for (int q = 0; q < MG; ++q) {
        if (q >= nm) break;
        const size_t o = ((size_t)c * M + m0 + q) * P::F + e0;
        const cpx v = conj_out ? cconj(dg[q]) : dg[q];
        dgrow[o] = accumulate ? cadd(dgrow[o], v) : v;
        if (srow) srow[o] = sum_acc ? cadd(srow[o], sg[q]) : sg[q];
    }
}

// dx, last stage: the inverse of sample b's dx half-spectrum with the unshifted roll
// (kernels_pallas.py:1798-1812); one wavefront per sample.
template <int FH, int FW>
__global__ __launch_bounds__(64) void k_pdx_half(int hin, int win, int ph, int pw, int ng,
                                                 const cpx* __restrict__ dxs,
                                                 float* __restrict__ dx) {
    using P = PGeo<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    cpx* T = reinterpret_cast<cpx*>(lds);
    const int lane = threadIdx.x, kc = lane >> 1, t = lane & 1;
    const int b = blockIdx.x;
    const cpx* src = dxs + (size_t)b * P::F;
    const size_t gs = (size_t)gridDim.x * P::F;  // the ng direction-group partials, in order
    auto at = [&](int e) {
        cpx a = src[e];
        for (int q = 1; q < ng; ++q) a = cadd(a, src[q * gs + e]);
        return a;
    };
    cpx v[P::HH];
#pragma unroll
    for (int j = 0; j < P::HH; ++j) v[j] = at((2 * j + t) * P::SP + kc);
    if (kc == 0) {  // packed column 0: DC + i*Nyquist
#pragma unroll
        for (int j = 0; j < P::HH; ++j) v[j] = cadd(v[j], cmul_i(at((2 * j + t) * P::SP + FW / 2)));
    }
    pcol_inv<FH, FW>(v, T);
    __syncthreads();
    prow_inv<FH, FW>(T, (FH - ph) & (FH - 1), (FW - pw) & (FW - 1), hin, 1.0f / (float)(FH * FW),
                     lds);
    __syncthreads();
    pstage_copy<FW>(lds, hin, win, dx + (size_t)b * hin * win);
}

// Forward correlation, one wavefront per plane g = b*M + m: z_bm = irfft2(xhat_b * ghat_m)
// read from row ph, column pw (kernels_pallas.py:1779-1791; kernels_greens.py:316-343).
template <int FH, int FW>
__global__ __launch_bounds__(64) void k_pconv_fwd(int M, int hout, int wout, int ph, int pw,
                                                  int nq_off, const cpx* __restrict__ xhat,
                                                  const cpx* __restrict__ ghat,
                                                  float* __restrict__ z) {
    using P = PGeo<FH, FW>;
    HIP_DYNAMIC_SHARED(float, lds)
    cpx* T = reinterpret_cast<cpx*>(lds);
    cpx* NQ = T + nq_off;
    const int lane = threadIdx.x, kc = lane >> 1, t = lane & 1;
    const int g = blockIdx.x, b = g / M, m = g - b * M;
    const cpx* X = xhat + (size_t)b * P::F;
    const cpx* G = ghat + (size_t)m * P::F;
    if (lane < FH) NQ[lane] = cmul(X[lane * P::SP + FW / 2], G[lane * P::SP + FW / 2]);
    cpx v[P::HH];
#pragma unroll
    for (int j = 0; j < P::HH; ++j) {
        const int e = (2 * j + t) * P::SP + kc;
        v[j] = cmul(X[e], G[e]);
    }
    __syncthreads();
    if (kc == 0) {
#pragma unroll
        for (int j = 0; j < P::HH; ++j) v[j] = cadd(v[j], cmul_i(NQ[2 * j + t]));
    }
    pcol_inv<FH, FW>(v, T);
    __syncthreads();
    prow_inv<FH, FW>(T, ph, pw, hout, 1.0f / (float)(FH * FW), lds);
    __syncthreads();
    pstage_copy<FW>(lds, hout, wout, z + (size_t)g * hout * wout);
}

// Forward correlation fused with the hidden-step epilogue (kernels_pallas.py:1779-1791 then
// 163-291): workgroup (b, g) of 4 wavefronts, wavefront w computing the plane m = 4g + w as
// k_pconv_fwd does (storing it to z when z is given), then its plane statistics (mean, then
// the centred sum of squares: population variance, eps 1e-5), zhat and act(zhat + b_roi).
// Each wavefront leaves zhat, then act, in its own LDS region; the workgroup adds the four in
// increasing m and writes the direction group's partial output
// parts[g][b] = w_eff * sum zhat + s_eff * sum act, the layout of nc_epilogue_fwd_parts.
// NE >= ceil(N / 64) plane values per lane (the full-row form: in runs of 4 consecutive
// pixels, 16-byte moves of b_roi and z when N % 4 == 0); every loop runs NE (or NE / 4) times
// with clamped loads, so a wavefront's loads issue together.
template <int FH, int FW, int ACT, int NE, bool WIN>
__global__ __launch_bounds__(256, 2) void k_pconv_epi(int B, int M, int hout, int wout, int ph,
                                                   int pw, int nq_off, int region, float slope,
                                                   const cpx* __restrict__ xhat,
                                                   const cpx* __restrict__ ghat,
                                                   const float* __restrict__ w_eff,
                                                   const float* __restrict__ s_eff,
                                                   const float* __restrict__ b_roi,
                                                   float* __restrict__ z,
                                                   float* __restrict__ parts,
                                                   float* __restrict__ mean,
                                                   float* __restrict__ rstd) {
    using P = PGeo<FH, FW>;
    constexpr int NC = NE / 4;  // output pixels per thread in the combine
    HIP_DYNAMIC_SHARED(float, ldsall)
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float* lds = ldsall + (size_t)wv * region;
    cpx* T = reinterpret_cast<cpx*>(lds);
    cpx* NQ = T + nq_off;
    const int b = blockIdx.x, g = blockIdx.y;
    // the idle wavefronts of the last group (4g + w >= M) repeat direction M - 1, store
    // nothing and leave zeros in their region, so control flow stays uniform
    const int m = min(g * 4 + wv, M - 1);
    const bool live = g * 4 + wv < M;
    const int N = hout * wout;
    const float inv_n = 1.0f / (float)N;
    const int kc = lane >> 1, t = lane & 1;
    const cpx* X = xhat + (size_t)b * P::F;
    const cpx* Gm = ghat + (size_t)m * P::F;
    if (lane < FH) NQ[lane] = cmul(X[lane * P::SP + FW / 2], Gm[lane * P::SP + FW / 2]);
    cpx v[P::HH];
#pragma unroll
    for (int j = 0; j < P::HH; ++j) {
        const int e = (2 * j + t) * P::SP + kc;
        v[j] = cmul(X[e], Gm[e]);
    }
    __syncthreads();
    if (kc == 0) {
#pragma unroll
        for (int j = 0; j < P::HH; ++j) v[j] = cadd(v[j], cmul_i(NQ[2 * j + t]));
    }
    if constexpr (WIN) {
        pcol_inv_rows<FH, FW>(v, T, ph, hout);
        __syncthreads();
        prow_inv<FH, FW>(T, 0, pw, hout, 1.0f / (float)(FH * FW), lds);
    } else {
        pcol_inv<FH, FW>(v, T);
        __syncthreads();
        prow_inv<FH, FW>(T, ph, pw, hout, 1.0f / (float)(FH * FW), lds);
    }
    __syncthreads();
    // the per-pixel parameters, requested together; their latency hides behind the statistics
    // plane value i of a lane is element pe(i): in the full-row form runs of 4 consecutive
    // pixels, moved as 16-byte loads and stores when the plane size and the operands allow
    // (in the windowed form, whose registers must leave room for three workgroups per CU,
    // element lane + 64 i)
    auto pe = [&](int i) {
        if constexpr (WIN) return lane + 64 * i;
        else return 4 * (lane + 64 * (i >> 2)) + (i & 3);
    };
    const bool v4 = !WIN && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(b_roi) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(z) & 15) == 0;
    float bv[NE], wq[NC], sq_[NC];
    if (v4) {
#pragma unroll
        for (int j = 0; j < NE / 4; ++j) {
            const float4 b4 =
                reinterpret_cast<const float4*>(b_roi)[min(lane + 64 * j, (N >> 2) - 1)];
            bv[4 * j] = b4.x;
            bv[4 * j + 1] = b4.y;
            bv[4 * j + 2] = b4.z;
            bv[4 * j + 3] = b4.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NE; ++i) bv[i] = b_roi[min(pe(i), N - 1)];
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int e = min((int)threadIdx.x + 256 * i, N - 1);
        wq[i] = w_eff[e];
        sq_[i] = s_eff[e];
    }
    // the plane, element e = pe(i) at (e / wout, e % wout) of the staging
    const unsigned inv = ((1u << 20) + wout - 1) / wout;
    float zv[NE];
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const int e = min(pe(i), N - 1);
        const int r = (int)(((unsigned)e * inv) >> 20);
        zv[i] = lds[r * (FW + 1) + (e - r * wout)];
    }
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) sum += pe(i) < N ? zv[i] : 0.f;
    if (z && live) {
        float* zo = z + ((size_t)b * M + m) * N;
        if (v4) {
#pragma unroll
            for (int j = 0; j < NE / 4; ++j)
                if (4 * (lane + 64 * j) < N)
                    reinterpret_cast<float4*>(zo)[lane + 64 * j] =
                        make_float4(zv[4 * j], zv[4 * j + 1], zv[4 * j + 2], zv[4 * j + 3]);
        } else {
#pragma unroll
            for (int i = 0; i < NE; ++i)
                if (pe(i) < N) zo[pe(i)] = zv[i];
        }
    }
    const float mu = wave_sum(sum) * inv_n;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const float d = pe(i) < N ? zv[i] - mu : 0.f;
        ss += d * d;
    }
    const float r = 1.0f / sqrtf(wave_sum(ss) * inv_n + 1e-5f);
    if (lane == 0 && live) {
        mean[(size_t)b * M + m] = mu;
        rstd[(size_t)b * M + m] = r;
    }
    // (zhat, act(zhat + b_roi)) replace the staging in this wavefront's region once every lane
    // has read it (WIN: zhat, then act, one plane of N floats at a time); the workgroup sums
    // each over its four directions in increasing m
    __syncthreads();
    const float on = live ? 1.f : 0.f;
    if constexpr (!WIN) {
        float* L = lds;
        float* A = lds + N;
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const int e = pe(i);
            const float zn = (zv[i] - mu) * r;
            const float a = act_f<ACT>(zn + bv[i], slope);
            if (e < N) {
                L[e] = zn * on;
                A[e] = a * on;
            }
        }
        __syncthreads();
        float* out = parts + ((size_t)g * B + b) * N;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int e = (int)threadIdx.x + 256 * i;
            const int ec = min(e, N - 1);
            float lin = ldsall[ec], ac = ldsall[N + ec];
#pragma unroll
            for (int q = 1; q < 4; ++q) {
                lin += ldsall[(size_t)q * region + ec];
                ac += ldsall[(size_t)q * region + N + ec];
            }
            if (e < N) out[e] = wq[i] * lin + sq_[i] * ac;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const int e = pe(i);
        zv[i] = (zv[i] - mu) * r;
        if (e < N) lds[e] = zv[i] * on;
    }
    __syncthreads();
    float lin[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int ec = min((int)threadIdx.x + 256 * i, N - 1);
        lin[i] = ldsall[ec];
#pragma unroll
        for (int q = 1; q < 4; ++q) lin[i] += ldsall[(size_t)q * region + ec];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const int e = pe(i);
        const float a = act_f<ACT>(zv[i] + bv[i], slope);
        if (e < N) lds[e] = a * on;
    }
    __syncthreads();
    float* out = parts + ((size_t)g * B + b) * N;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int e = (int)threadIdx.x + 256 * i;
        const int ec = min(e, N - 1);
        float ac = ldsall[ec];
#pragma unroll
        for (int q = 1; q < 4; ++q) ac += ldsall[(size_t)q * region + ec];
        if (e < N) out[e] = wq[i] * lin[i] + sq_[i] * ac;
    }
}

// Forward correlation fused with the output-port statistics (kernels_pallas.py:1779-1791
// then 1284-1347 and 1510-1551): workgroup (b, g) of 4 wavefronts, wavefront w correlating the
// plane m = 4g + w (stored to z when z is given) and forming its mean and centred variance
// (population, eps 1e-5), then zo[b][m][k] = (z[port_idx[k]] - mean) rstd for the P port
// cells.  The workgroup adds its directions' zo (increasing m) into the partial sums
// part (2, G, B, P) = (Σ zo, Σ final_act(zo + b_out)) that k_port_combine turns into the
// port outputs, as nc_port_fwd's split does.  The idle wavefronts of the last group repeat
// m = M - 1 and store nothing.
template <int FH, int FW, int NE, bool WIN>
__global__ __launch_bounds__(256, 2) void k_pconv_port(int B, int M, int hout, int wout, int ph,
                                                    int pw, int nq_off, int region, int P,
                                                    int fact, float slope,
                                                    const cpx* __restrict__ xhat,
                                                    const cpx* __restrict__ ghat,
                                                    const int* __restrict__ pidx,
                                                    const float* __restrict__ pp,
                                                    float* __restrict__ z,
                                                    float* __restrict__ zo,
                                                    float* __restrict__ mean,
                                                    float* __restrict__ rstd,
                                                    float* __restrict__ part) {
    using P_ = PGeo<FH, FW>;
    constexpr int PK = 4;  // port cells per lane (P <= 256)
    HIP_DYNAMIC_SHARED(float, ldsall)
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float* lds = ldsall + (size_t)wv * region;
    cpx* T = reinterpret_cast<cpx*>(lds);
    cpx* NQ = T + nq_off;
    const int b = blockIdx.x, g = blockIdx.y;
    const int m = min(g * 4 + wv, M - 1), nm = min(4, M - g * 4);
    const bool live = g * 4 + wv < M;
    const int N = hout * wout;
    const float inv_n = 1.0f / (float)N;
    const int kc = lane >> 1, t = lane & 1;
    const cpx* X = xhat + (size_t)b * P_::F;
    const cpx* Gm = ghat + (size_t)m * P_::F;
    if (lane < FH) NQ[lane] = cmul(X[lane * P_::SP + FW / 2], Gm[lane * P_::SP + FW / 2]);
    cpx v[P_::HH];
#pragma unroll
    for (int j = 0; j < P_::HH; ++j) {
        const int e = (2 * j + t) * P_::SP + kc;
        v[j] = cmul(X[e], Gm[e]);
    }
    __syncthreads();
    if (kc == 0) {
#pragma unroll
        for (int j = 0; j < P_::HH; ++j) v[j] = cadd(v[j], cmul_i(NQ[2 * j + t]));
    }
    if constexpr (WIN) {
        pcol_inv_rows<FH, FW>(v, T, ph, hout);
        __syncthreads();
        prow_inv<FH, FW>(T, 0, pw, hout, 1.0f / (float)(FH * FW), lds);
    } else {
        pcol_inv<FH, FW>(v, T);
        __syncthreads();
        prow_inv<FH, FW>(T, ph, pw, hout, 1.0f / (float)(FH * FW), lds);
    }
    __syncthreads();
    // the port cells' flat indices, requested before the statistics
    int pe[PK];
#pragma unroll
    for (int j = 0; j < PK; ++j) pe[j] = min(max(pidx[min(lane + 64 * j, P - 1)], 0), N - 1);
    // plane value i of a lane is element px(i): in the full-row form runs of 4 consecutive
    // pixels, z stored as 16-byte moves when the plane size and z allow (in the windowed form
    // element lane + 64 i)
    auto px = [&](int i) {
        if constexpr (WIN) return lane + 64 * i;
        else return 4 * (lane + 64 * (i >> 2)) + (i & 3);
    };
    const bool v4 = !WIN && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(z) & 15) == 0;
    const unsigned inv = ((1u << 20) + wout - 1) / wout;
    float zv[NE];
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const int e = min(px(i), N - 1);
        const int r = (int)(((unsigned)e * inv) >> 20);
        zv[i] = lds[r * (FW + 1) + (e - r * wout)];
    }
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) sum += px(i) < N ? zv[i] : 0.f;
    if (z && live) {
        float* zp = z + ((size_t)b * M + m) * N;
        if (v4) {
#pragma unroll
            for (int j = 0; j < NE / 4; ++j)
                if (4 * (lane + 64 * j) < N)
                    reinterpret_cast<float4*>(zp)[lane + 64 * j] =
                        make_float4(zv[4 * j], zv[4 * j + 1], zv[4 * j + 2], zv[4 * j + 3]);
        } else {
#pragma unroll
            for (int i = 0; i < NE; ++i)
                if (px(i) < N) zp[px(i)] = zv[i];
        }
    }
    const float mu = wave_sum(sum) * inv_n;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const float d = px(i) < N ? zv[i] - mu : 0.f;
        ss += d * d;
    }
    const float r = 1.0f / sqrtf(wave_sum(ss) * inv_n + 1e-5f);
    if (lane == 0 && live) {
        mean[(size_t)b * M + m] = mu;
        rstd[(size_t)b * M + m] = r;
    }
    float pz[PK];
#pragma unroll
    for (int j = 0; j < PK; ++j) {
        const int rr = (int)(((unsigned)pe[j] * inv) >> 20);
        pz[j] = (lds[rr * (FW + 1) + (pe[j] - rr * wout)] - mu) * r;
    }
    // zo, and the wavefront's zo in its region for the direction sums, once every lane has
    // read the staging
    __syncthreads();
    float* zop = zo + ((size_t)b * M + m) * P;
#pragma unroll
    for (int j = 0; j < PK; ++j) {
        const int k = lane + 64 * j;
        if (k < P) {
            if (live) zop[k] = pz[j];
            lds[k] = pz[j];
        }
    }
    __syncthreads();
    const size_t GBP = (size_t)gridDim.y * B * P;
    for (int k = threadIdx.x; k < P; k += blockDim.x) {
        const float bo = pp[2 * P + k];
        float lin = 0.f, ac = 0.f;
        for (int q = 0; q < nm; ++q) {
            const float u = ldsall[(size_t)q * region + k];
            lin += u;
            if (fact != NC_ACT_IDENTITY) ac += nc_act(u + bo, fact, slope);
        }
        part[((size_t)g * B + b) * P + k] = lin;
        part[GBP + ((size_t)g * B + b) * P + k] = ac;
    }
}

// ----------------------------------------------------------------------------------------
// Launch plumbing
// ----------------------------------------------------------------------------------------

bool pow2_ok(int f) { return f == 16 || f == 32 || f == 64; }

// LDS of a wavefront transform over `rows` rows of PPW planes: the transposition buffer T
// (rows + 2 with the trash and zero rows) and the real-valued staging (input or output), which
// shares T's space when one row pass covers every row pair; then the Nyquist-column staging
// (PPW x FH cpx).
template <int FH, int FW>
struct WLds {
    size_t bytes;
    int off;  // float offset of the staging area
    int nq;   // cpx offset of the Nyquist staging
    WLds(int rows, int cols, size_t at_least = 0) {
        using W = WGeo<FH, FW>;
        const size_t t = (size_t)W::PPW * (rows + 2) * W::PITCH * sizeof(cpx);
        const size_t st = (size_t)std::max(ostage_floats(W::PPW, rows, FW),
                                           istage_floats(W::PPW, rows, FW)) * sizeof(float);
        const bool share = W::PPW * ((rows + 1) / 2) <= 64;
        size_t main = std::max(share ? std::max(t, st) : t + st, at_least);
        main = (main + 15) / 16 * 16;
        off = share ? 0 : (int)(t / sizeof(float));
        nq = (int)(main / sizeof(cpx));
        bytes = main + (size_t)W::PPW * FH * sizeof(cpx);
    }
};

// float4 moves need 16-byte aligned planes.
inline int vec_ok(const void* p, size_t n) {
    return (n % 4 == 0) && (reinterpret_cast<uintptr_t>(p) % 16 == 0);
}

// Compute units of the current device (queried once per device).
int cu_count() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <class K>
void lds_limit(K kernel, size_t bytes) {
    if (bytes > 65536)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

// Direction groups of the backward: each wavefront transforms PPW planes of one sample.
template <int FH, int FW>
int bwd_groups(int M) {
    constexpr int PPW = WGeo<FH, FW>::PPW;
    return (M + PPW - 1) / PPW;
}

// Sample chunks of the dG reduction.  Lane-pair grids (the fused k_pbwd_red): chunks of
// kPChunk samples, which measured best against the larger row stacks they leave.  Otherwise
// enough threads (about 2^18) to keep HBM busy, at most one load batch per chunk.
constexpr int kPChunk = 8;

template <int FH, int FW>
int dg_chunks(int B, int M) {
    if (pair_grid<FH, FW>()) return std::max(1, (B + kPChunk - 1) / kPChunk);
    const int per = M * WGeo<FH, FW>::F;
    const int by_threads = (262144 + per - 1) / per;
    const int by_batch = (B + kDgBatch - 1) / kDgBatch;  // at most one load batch per chunk
    return std::max(1, std::min(B, std::max(by_threads, by_batch)));
}

// Workspace: dx partials (B, MG, PF), their sums (B, PF), the cotangent half-spectra
// (M, B, pitch) and the dG chunk partials (chunks, M, F).
template <int FH, int FW>
size_t bwd_ws(int B, int M) {
    if constexpr (pair_grid<FH, FW>()) {
        // cotangent half-spectra (M, B, pitch), dx spectra (B, F), dG and spectrum-sum chunk
        // rows
        using P = PGeo<FH, FW>;
        const size_t nc = dg_chunks<FH, FW>(B, M);
        return ((size_t)M * B * spec_pitch<FH, FW>() + (size_t)B * P::F + 2 * nc * M * P::F) *
               sizeof(cpx);
    }
    using W = WGeo<FH, FW>;
    const size_t mg = bwd_groups<FH, FW>(M);
    const size_t nc = dg_chunks<FH, FW>(B, M);
    return (((size_t)B * mg + (size_t)B) * W::PF + (size_t)M * B * spec_pitch<FH, FW>() +
            2 * nc * M * W::F) * sizeof(cpx);
}

// Sample chunks the dG reduction actually launches (its partial rows).
template <int FH, int FW>
int dg_parts(int B, int M) {
    const int nchunk = dg_chunks<FH, FW>(B, M);
    const int bper = (B + nchunk - 1) / nchunk;
    return (B + bper - 1) / bper;
}

// The dG (and spectrum-sum) reduction over the stored cotangent spectra: into dghat / ssum
// through the chunk partials dgpart and k_wbwd_dg_sum, or, parts_mode, into their row stacks.
template <int FH, int FW>
int launch_dg(hipStream_t st, int B, int M, const cpx* spec, const float* xhat, float* dghat,
              int accumulate, int conj_out, float* ssum, int sum_acc, cpx* dgpart,
              bool parts_mode) {
    constexpr int F = WGeo<FH, FW>::F;
    const int nb = dg_parts<FH, FW>(B, M);
    const int bper = (B + nb - 1) / nb;
    cpx* sc = reinterpret_cast<cpx*>(ssum);
    hipLaunchKernelGGL((k_wbwd_dg_red<FH, FW>), dim3((F + 255) / 256, M, nb), dim3(256), 0, st, B,
                       M, bper, spec, reinterpret_cast<const cpx*>(xhat), dgpart,
                       reinterpret_cast<cpx*>(dghat), accumulate, conj_out, sc, sum_acc,
                       parts_mode ? 1 : 0);
    NC_CHECK_LAUNCH();
    if (nb > 1 && !parts_mode) {
        hipLaunchKernelGGL(k_wbwd_dg_sum, dim3((F + 255) / 256, M, sc ? 2 : 1), dim3(256), 0, st,
                           nb, M, F, dgpart, reinterpret_cast<cpx*>(dghat), accumulate, conj_out,
                           sc, sum_acc);
        NC_CHECK_LAUNCH();
    }
    return NC_OK;
}

template <int FH, int FW, bool FLIP, int POST, int NP>
void launch_rfft2_k(hipStream_t st, int nplanes, int hin, int win, const float* x, cpx* out,
                    const SpecPost& post, size_t qstride, int nq) {
    const int vec = vec_ok(x, (size_t)hin * win) && (nq == 1 || qstride % 4 == 0);
    if constexpr (pair_grid<FH, FW>()) {
        const PLds l(hin, PGeo<FH, FW>::PITCH, FW, FH, false);
        lds_limit(k_prfft2<FH, FW, FLIP, POST, NP>, l.bytes);
        hipLaunchKernelGGL((k_prfft2<FH, FW, FLIP, POST, NP>), dim3(nplanes), dim3(64), l.bytes,
                           st, hin, win, vec, x, out, post, qstride, nq);
    } else {
        using W = WGeo<FH, FW>;
        WLds<FH, FW> l(hin, win);
        lds_limit(k_wrfft2<FH, FW, FLIP, POST, NP>, l.bytes);
        hipLaunchKernelGGL((k_wrfft2<FH, FW, FLIP, POST, NP>),
                           dim3((nplanes + W::PPW - 1) / W::PPW), dim3(64), l.bytes, st, nplanes,
                           hin, win, l.off, vec, x, out, post, qstride, nq);
    }
}

template <int FH, int FW, int NP>
void launch_rfft2_np(hipStream_t st, int nplanes, int hin, int win, const float* x, cpx* out,
                     int post_kind, const SpecPost& post, size_t qstride, int nq) {
    if (post_kind == kPostAdd)
        launch_rfft2_k<FH, FW, false, kPostAdd, NP>(st, nplanes, hin, win, x, out, post, qstride,
                                                    nq);
    else if (post_kind == kPostShift)
        launch_rfft2_k<FH, FW, false, kPostShift, NP>(st, nplanes, hin, win, x, out, post,
                                                      qstride, nq);
    else
        launch_rfft2_k<FH, FW, false, kPostNone, NP>(st, nplanes, hin, win, x, out, post,
                                                     qstride, nq);
}

// k_r8rfft2 over nplanes planes of at most 64 x 64 (nparts partial planes each).
template <int POST>
void launch_r8rfft2(hipStream_t st, int nplanes, int hin, int win, const float* x, cpx* out,
                    const SpecPost& post, int nparts, size_t qstride) {
#define NC_R8(NP_)                                                                          \
    do {                                                                                    \
        lds_limit(k_r8rfft2<POST, NP_>, r8::kFwdLdsBytes);                                  \
        hipLaunchKernelGGL((k_r8rfft2<POST, NP_>), dim3(nplanes), dim3(r8::kNT),            \
                           r8::kFwdLdsBytes, st, hin, win, qstride, nparts, x, out, post); \
    } while (0)
    if (nparts == 1) NC_R8(1);
    else if (nparts == 4) NC_R8(4);
    else NC_R8(0);
#undef NC_R8
}

// Half-spectra of nplanes real planes; flip (the filter spectra) takes no post-operation.
// nparts > 1: each plane is the sum of nparts partial planes qstride floats apart.
template <int FH, int FW>
int launch_rfft2(hipStream_t st, int nplanes, int hin, int win, bool flip, const float* x,
                 cpx* out, int post_kind = kPostNone, const SpecPost& post = SpecPost{},
                 int nparts = 1, size_t qstride = 0) {
    if constexpr (seg_grid<FH, FW>()) {
        // unflipped planes without a phase ramp: one radix-8 workgroup per plane once there
        // are more planes than CUs; below that the segmented transform's two column segments
        // per plane give the CUs more workgroups (config 0, 128 planes: 7.19 -> 7.12 us)
        if (!flip && post_kind != kPostShift && nplanes > cu_count()) {
            if (post_kind == kPostAdd)
                launch_r8rfft2<kPostAdd>(st, nplanes, hin, win, x, out, post, nparts, qstride);
            else
                launch_r8rfft2<kPostNone>(st, nplanes, hin, win, x, out, post, nparts, qstride);
            NC_CHECK_LAUNCH();
            return NC_OK;
        }
        return nc_seg_rfft2(st, FH, FW, nplanes, hin, win, flip ? 1 : 0, x, out,
                            post_kind == kPostAdd ? post.add : nullptr,
                            post_kind == kPostShift ? post.sh : 0,
                            post_kind == kPostShift ? post.sw : 0, nparts, qstride);
    }
    if (flip)
        launch_rfft2_k<FH, FW, true, kPostNone, 1>(st, nplanes, hin, win, x, out, post, 0, 1);
    else if (nparts == 1)
        launch_rfft2_np<FH, FW, 1>(st, nplanes, hin, win, x, out, post_kind, post, 0, 1);
    else if (nparts == 4 && pair_grid<FH, FW>())
        launch_rfft2_np<FH, FW, 4>(st, nplanes, hin, win, x, out, post_kind, post, qstride, 4);
    else
        launch_rfft2_np<FH, FW, 0>(st, nplanes, hin, win, x, out, post_kind, post, qstride,
                                   nparts);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

// z_bm = irfft2(xhat_b * ghat_m), the (hout, wout) window from (ph, pw).
template <int FH, int FW>
int launch_corr(hipStream_t st, int B, int M, int hout, int wout, int ph, int pw,
                const float* xhat, const float* ghat, float* z) {
    using W = WGeo<FH, FW>;
    if constexpr (pair_grid<FH, FW>()) {
        const PLds l(hout, PGeo<FH, FW>::PITCH, FW, FH, true);
        lds_limit(k_pconv_fwd<FH, FW>, l.bytes);
        hipLaunchKernelGGL((k_pconv_fwd<FH, FW>), dim3(B * M), dim3(64), l.bytes, st, M, hout,
                           wout, ph, pw, l.nq, reinterpret_cast<const cpx*>(xhat),
                           reinterpret_cast<const cpx*>(ghat), z);
        NC_CHECK_LAUNCH();
        return NC_OK;
    }
    WLds<FH, FW> l(hout, wout);
    lds_limit(k_wconv_fwd<FH, FW>, l.bytes);
    const int nplanes = B * M;
    hipLaunchKernelGGL((k_wconv_fwd<FH, FW>), dim3((nplanes + W::PPW - 1) / W::PPW), dim3(64),
                       l.bytes, st, nplanes, M, hout, wout, ph, pw, l.off, l.nq,
                       vec_ok(z, (size_t)hout * wout),
                       reinterpret_cast<const cpx*>(xhat), reinterpret_cast<const cpx*>(ghat), z);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

// Per-wavefront LDS region (floats) of the fused correlation + hidden epilogue: the inverse
// transform's staging, or the plane's (zhat, act) pair, whichever is larger; WIN: the staging
// over the output window's rows only (pcol_inv_rows), or one plane (zhat, then act).  0 when
// four regions do not fit one workgroup's LDS.
template <int FH, int FW>
int corr_epi_region(int hout, int wout, bool win = false) {
    const PLds l(hout, PGeo<FH, FW>::PITCH, FW, FH, true, win);
    const size_t fl = std::max(l.bytes / sizeof(float), (size_t)(win ? 1 : 2) * hout * wout);
    const size_t region = (fl + 15) / 16 * 16;
    return 4 * region * sizeof(float) <= 163840 ? (int)region : 0;
}

int corr_epi_region(int fft_h, int fft_w, int hout, int wout) {
    if (fft_w != 64 || hout <= 0 || wout <= 0 || hout > fft_h || wout > fft_w) return 0;
    if (fft_h == 64) return corr_epi_region<64, 64>(hout, wout);
    if (fft_h == 32) return corr_epi_region<32, 64>(hout, wout);
    return 0;
}

// The windowed form of the fused kernels (a smaller LDS region: three workgroups per CU
// instead of two) for grids of more than two workgroups per CU.  At two or fewer per CU its
// extra barriers and predicated stores cost more than the occupancy gains (config 0: 25.0 ->
// 27.3 us per hidden step), while a B = 1024 evaluation gains a fifth in throughput.
bool corr_windowed(const dim3& grid) {
    return (size_t)grid.x * grid.y > 2 * (size_t)cu_count();
}

// The fused correlation + hidden epilogue on the lane-pair grids; false when the plane is
// too large for the per-wavefront LDS region (the caller falls back).
template <int FH, int FW>
bool launch_corr_epi(hipStream_t st, int B, int M, int hout, int wout, int ph, int pw, int act,
                     float slope, const float* xhat, const float* ghat, const float* w_eff,
                     const float* s_eff, const float* b_roi, float* z, float* parts,
                     float* mean, float* rstd) {
    if constexpr (!pair_grid<FH, FW>()) {
        return false;
    } else {
        if (corr_epi_region<FH, FW>(hout, wout) == 0) return false;
        const dim3 grid(B, (M + 3) / 4);
        const bool win = corr_windowed(grid);
        const PLds l(hout, PGeo<FH, FW>::PITCH, FW, FH, true, win);
        const int region = corr_epi_region<FH, FW>(hout, wout, win);
        const size_t bytes = (size_t)4 * region * sizeof(float);
        const int N = hout * wout;
#define NC_CE3(A_, NE_, W_)                                                                    \
    do {                                                                                       \
        lds_limit(k_pconv_epi<FH, FW, A_, NE_, W_>, bytes);                                    \
        hipLaunchKernelGGL((k_pconv_epi<FH, FW, A_, NE_, W_>), grid, dim3(256), bytes, st, B,  \
                           M, hout, wout, ph, pw, l.nq, region, slope,                         \
                           reinterpret_cast<const cpx*>(xhat),                                 \
                           reinterpret_cast<const cpx*>(ghat), w_eff, s_eff, b_roi, z, parts,  \
                           mean, rstd);                                                        \
    } while (0)
#define NC_CE2(A_, NE_)                         \
    do {                                        \
        if (win) NC_CE3(A_, NE_, true);         \
        else NC_CE3(A_, NE_, false);            \
    } while (0)
#define NC_CE(A_)                                                        \
    do {                                                                 \
        if (FH * FW > 2048 && N > 2048) NC_CE2(A_, FH * FW / 64);       \
        else NC_CE2(A_, 32);                                             \
    } while (0)
        switch (act) {
            case NC_ACT_TANH: NC_CE(NC_ACT_TANH); break;
            case NC_ACT_SIGMOID: NC_CE(NC_ACT_SIGMOID); break;
            case NC_ACT_RELU: NC_CE(NC_ACT_RELU); break;
            case NC_ACT_LEAKY_RELU: NC_CE(NC_ACT_LEAKY_RELU); break;
            case NC_ACT_GELU: NC_CE(NC_ACT_GELU); break;
            default: NC_CE(NC_ACT_IDENTITY);
        }
#undef NC_CE
#undef NC_CE2
#undef NC_CE3
        return true;
    }
}

template <int FH, int FW>
bool launch_corr_port(hipStream_t st, int B, int M, int hout, int wout, int ph, int pw, int P,
                      int fact, float slope, const float* xhat, const float* ghat,
                      const int32_t* pidx, const float* pp, float* z, float* zo, float* mean,
                      float* rstd, float* part) {
    if constexpr (!pair_grid<FH, FW>()) {
        return false;
    } else {
        const int full = corr_epi_region<FH, FW>(hout, wout);
        if (full == 0 || full < P) return false;
        const dim3 grid(B, (M + 3) / 4);
        const bool win = corr_windowed(grid) && corr_epi_region<FH, FW>(hout, wout, true) >= P;
        const PLds l(hout, PGeo<FH, FW>::PITCH, FW, FH, true, win);
        const int region = win ? corr_epi_region<FH, FW>(hout, wout, true) : full;
        const size_t bytes = (size_t)4 * region * sizeof(float);
#define NC_CP2(NE_, W_)                                                                       \
    do {                                                                                      \
        lds_limit(k_pconv_port<FH, FW, NE_, W_>, bytes);                                      \
        hipLaunchKernelGGL((k_pconv_port<FH, FW, NE_, W_>), grid, dim3(256), bytes, st, B, M, \
                           hout, wout, ph, pw, l.nq, region, P, fact, slope,                  \
                           reinterpret_cast<const cpx*>(xhat),                                \
                           reinterpret_cast<const cpx*>(ghat), pidx, pp, z, zo, mean, rstd,   \
                           part);                                                             \
    } while (0)
#define NC_CP(NE_)                     \
    do {                               \
        if (win) NC_CP2(NE_, true);    \
        else NC_CP2(NE_, false);       \
    } while (0)
        if (FH * FW > 2048 && hout * wout > 2048) NC_CP(FH * FW / 64);
        else NC_CP(32);
#undef NC_CP
#undef NC_CP2
        return true;
    }
}

template <int FH, int FW>
int launch_fwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout, int ph,
               int pw, const float* x, int nparts, const float* xhat_add, const float* ghat,
               float* z, float* xhat) {
    const SpecPost post{reinterpret_cast<const cpx*>(xhat_add), 0, 0};
    int rc = launch_rfft2<FH, FW>(st, B, hin, win, false, x, reinterpret_cast<cpx*>(xhat),
                                  xhat_add ? kPostAdd : kPostNone, post, nparts,
                                  (size_t)B * hin * win);
    if (rc != NC_OK) return rc;
    return launch_corr<FH, FW>(st, B, M, hout, wout, ph, pw, xhat, ghat, z);
}

// Several independent spectrum jobs (nc_plane_spectra) in one launch: block g runs plane
// g - start[q] of the job q whose range holds g; each job's kind picks the transform variant.
constexpr int kMaxSpecJobs = 4;
struct SpecJobs {
    const float* x[kMaxSpecJobs];
    cpx* out[kMaxSpecJobs];
    SpecPost post[kMaxSpecJobs];
    int hin[kMaxSpecJobs], win[kMaxSpecJobs], vec[kMaxSpecJobs], kind[kMaxSpecJobs];
    int start[kMaxSpecJobs + 1];
    int n;
};
enum { kJobPlain = 0, kJobFlip = 1, kJobAdd = 2, kJobShift = 3 };

template <int FH, int FW>
__global__ __launch_bounds__(64) void k_pspectra(SpecJobs J) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int g = blockIdx.x;
    int q = 0;
    while (q + 1 < J.n && g >= J.start[q + 1]) ++q;
    const int i = g - J.start[q], hin = J.hin[q], win = J.win[q], vec = J.vec[q];
    const float* src = J.x[q] + (size_t)i * hin * win;
    cpx* o = J.out[q] + (size_t)i * PGeo<FH, FW>::F;
    switch (J.kind[q]) {
        case kJobFlip:
            prfft2_plane<FH, FW, true, kPostNone>(src, hin, win, vec, lds, o, J.post[q]);
            break;
        case kJobAdd:
            prfft2_plane<FH, FW, false, kPostAdd>(src, hin, win, vec, lds, o, J.post[q]);
            break;
        case kJobShift:
            prfft2_plane<FH, FW, false, kPostShift>(src, hin, win, vec, lds, o, J.post[q]);
            break;
        default:
            prfft2_plane<FH, FW, false, kPostNone>(src, hin, win, vec, lds, o, J.post[q]);
    }
}

template <int FH, int FW>
int launch_spectra(hipStream_t st, int n, const nc_spectrum_job* jobs) {
    if constexpr (seg_grid<FH, FW>()) {
        return nc_large_plane_spectra(st, FH, FW, n, jobs);
    } else if constexpr (pair_grid<FH, FW>()) {
        SpecJobs J{};
        J.n = n;
        size_t lds = 0;
        for (int q = 0; q < n; ++q) {
            const nc_spectrum_job& j = jobs[q];
            J.x[q] = j.x;
            J.out[q] = reinterpret_cast<cpx*>(j.xhat);
            J.post[q] = SpecPost{reinterpret_cast<const cpx*>(j.add), j.shift_h, j.shift_w};
            J.hin[q] = j.hin;
            J.win[q] = j.win;
            J.vec[q] = vec_ok(j.x, (size_t)j.hin * j.win);
            J.kind[q] = j.flip ? kJobFlip : j.add ? kJobAdd : (j.shift_h | j.shift_w) ? kJobShift
                                                                                       : kJobPlain;
            J.start[q + 1] = J.start[q] + j.nplanes;
            lds = std::max(lds, PLds(j.hin, PGeo<FH, FW>::PITCH, FW, FH, false).bytes);
        }
        lds_limit(k_pspectra<FH, FW>, lds);
        hipLaunchKernelGGL((k_pspectra<FH, FW>), dim3(J.start[n]), dim3(64), lds, st, J);
        NC_CHECK_LAUNCH();
        return NC_OK;
    }
    for (int q = 0; q < n; ++q) {  // wavefront grids: one launch per job
        const nc_spectrum_job& j = jobs[q];
        const SpecPost post{reinterpret_cast<const cpx*>(j.add), j.shift_h, j.shift_w};
        const int kind = j.add ? kPostAdd : (j.shift_h | j.shift_w) ? kPostShift : kPostNone;
        const int rc = launch_rfft2<FH, FW>(st, j.nplanes, j.hin, j.win, j.flip != 0, j.x,
                                            reinterpret_cast<cpx*>(j.xhat), kind, post);
        if (rc != NC_OK) return rc;
    }
    return NC_OK;
}

template <int FH, int FW>
int launch_pbwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout, int ph,
                int pw, const float* gz, const float* xhat, const float* ghat, int need_dx,
                float* dx, float* dghat, int accumulate, int conj_out, float* ssum, int sum_acc,
                bool parts_mode, void* ws) {
    using P = PGeo<FH, FW>;
    const int nb = dg_parts<FH, FW>(B, M);
    const int bper = (B + nb - 1) / nb;
    cpx* spec = reinterpret_cast<cpx*>(ws);
    cpx* dxs = spec + (size_t)M * B * spec_pitch<FH, FW>();
    cpx* rows = dxs + (size_t)B * P::F;  // chunk rows when they are not the caller's
    if constexpr (FH == 64) {
        lds_limit(k_r8spec, r8::kFwdLdsBytes);
        hipLaunchKernelGGL(k_r8spec, dim3(B * M), dim3(r8::kNT), r8::kFwdLdsBytes, st, B, M,
                           hout, wout, gz, spec);
    } else {
        const PLds ls(hout, P::PITCH, FW, FH, false);
        lds_limit(k_pspec<FH, FW>, ls.bytes);
        hipLaunchKernelGGL((k_pspec<FH, FW>), dim3(B * M), dim3(64), ls.bytes, st, B, M, hout,
                           wout, vec_ok(gz, (size_t)hout * wout), gz, spec);
    }
    NC_CHECK_LAUNCH();
    // the chunk rows: the caller's row stacks, the outputs themselves (one chunk), or the
    // workspace rows summed below
    const bool direct = parts_mode || nb == 1;
    cpx* dgr = direct ? reinterpret_cast<cpx*>(dghat) : rows;
    cpx* sr = ssum ? (direct ? reinterpret_cast<cpx*>(ssum) : rows + (size_t)nb * M * P::F)
                   : nullptr;
    // four waves per workgroup, MG = ceil(M / 4) directions each
    const dim3 grid((P::F + 63) / 64, nb);
#define NC_PBWD(MG_)                                                                            \
    hipLaunchKernelGGL((k_pbwd_red<FH, FW, MG_>), grid, dim3(256), 0, st, B, M, bper, need_dx,  \
                       spec, reinterpret_cast<const cpx*>(xhat),                                \
                       reinterpret_cast<const cpx*>(ghat), dxs, dgr, direct ? accumulate : 0,   \
                       direct ? conj_out : 0, sr, direct ? sum_acc : 0)
    if (M <= 4) NC_PBWD(1);
    else if (M <= 8) NC_PBWD(2);
    else if (M <= 16) NC_PBWD(4);
    else if (M <= 32) NC_PBWD(8);
    else if (M <= 64) NC_PBWD(16);
    else return NC_ERR_UNSUPPORTED;  // more directions than the epilogues take (kMaxM)
#undef NC_PBWD
    NC_CHECK_LAUNCH();
    if (!direct) {
        hipLaunchKernelGGL(k_wbwd_dg_sum, dim3((P::F + 255) / 256, M, ssum ? 2 : 1), dim3(256), 0,
                           st, nb, M, P::F, rows, reinterpret_cast<cpx*>(dghat), accumulate,
                           conj_out, reinterpret_cast<cpx*>(ssum), sum_acc);
        NC_CHECK_LAUNCH();
    }
    if (need_dx) {
        if constexpr (seg_grid<FH, FW>()) {
            const int rc = nc_seg_dx(st, B, 1, hin, win, ph, pw, FH, FW, dxs, dx);
            if (rc != NC_OK) return rc;
        } else {
            const PLds lf(hin, P::PITCH, FW, FH, true);
            lds_limit(k_pdx_half<FH, FW>, lf.bytes);
            hipLaunchKernelGGL((k_pdx_half<FH, FW>), dim3(B), dim3(64), lf.bytes, st, hin, win,
                               ph, pw, 1, dxs, dx);
            NC_CHECK_LAUNCH();
        }
    }
    return NC_OK;
}

template <int FH, int FW>
int launch_bwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout, int ph,
               int pw, const float* gz, const float* xhat, const float* ghat, int need_dx,
               float* dx, float* dghat, int accumulate, int conj_out, float* ssum, int sum_acc,
               bool parts_mode, void* ws) {
    if constexpr (pair_grid<FH, FW>())
        return launch_pbwd<FH, FW>(st, B, M, hin, win, hout, wout, ph, pw, gz, xhat, ghat, need_dx,
                                   dx, dghat, accumulate, conj_out, ssum, sum_acc, parts_mode,
                                   ws);
    using W = WGeo<FH, FW>;
    const int mg = bwd_groups<FH, FW>(M);
    cpx* dxpart = reinterpret_cast<cpx*>(ws);
    cpx* dxsum = dxpart + (size_t)B * mg * W::PF;
    cpx* spec = dxsum + (size_t)B * W::PF;
    const WLds<FH, FW> lp(hout, wout, (size_t)64 * (FH / 2) * sizeof(cpx));
    lds_limit(k_wbwd_part<FH, FW>, lp.bytes);
    hipLaunchKernelGGL((k_wbwd_part<FH, FW>), dim3(mg, B), dim3(64), lp.bytes, st, B, M, hout,
                       wout, lp.off, lp.nq, vec_ok(gz, (size_t)hout * wout), need_dx, gz,
                       reinterpret_cast<const cpx*>(ghat), dxpart, spec);
    NC_CHECK_LAUNCH();
    if (need_dx) {
        hipLaunchKernelGGL(k_psum, dim3((W::PF + 255) / 256, B), dim3(256), 0, st, mg, W::PF,
                           (size_t)mg * W::PF, (size_t)W::PF, dxpart, dxsum);
        NC_CHECK_LAUNCH();
        const WLds<FH, FW> lf(hin, win);
        lds_limit(k_wbwd_dx_fin<FH, FW>, lf.bytes);
        hipLaunchKernelGGL((k_wbwd_dx_fin<FH, FW>), dim3((B + W::PPW - 1) / W::PPW), dim3(64),
                           lf.bytes, st, B, hin, win, ph, pw, lf.off,
                           vec_ok(dx, (size_t)hin * win), dxsum, dx);
        NC_CHECK_LAUNCH();
    }
    cpx* dgpart = spec + (size_t)M * B * spec_pitch<FH, FW>();
    return launch_dg<FH, FW>(st, B, M, spec, xhat, dghat, accumulate, conj_out, ssum, sum_acc,
                             dgpart, parts_mode);
}

// Inverse of a one-sample dx spectrum (unpacked for the lane-pair grids, packed otherwise, as
// k_hat_red wrote it) with the unshifted roll.
template <int FH, int FW>
int launch_hat_dx(hipStream_t st, int hin, int win, int ph, int pw, const cpx* dxs, float* dx) {
    if constexpr (seg_grid<FH, FW>()) {
        return nc_seg_dx(st, 1, 1, hin, win, ph, pw, FH, FW, dxs, dx);
    } else if constexpr (pair_grid<FH, FW>()) {
        const PLds lf(hin, PGeo<FH, FW>::PITCH, FW, FH, true);
        lds_limit(k_pdx_half<FH, FW>, lf.bytes);
        hipLaunchKernelGGL((k_pdx_half<FH, FW>), dim3(1), dim3(64), lf.bytes, st, hin, win, ph,
                           pw, 1, dxs, dx);
        NC_CHECK_LAUNCH();
        return NC_OK;
    }
    const WLds<FH, FW> lf(hin, win);
    lds_limit(k_wbwd_dx_fin<FH, FW>, lf.bytes);
    hipLaunchKernelGGL((k_wbwd_dx_fin<FH, FW>), dim3(1), dim3(64), lf.bytes, st, 1, hin, win, ph,
                       pw, lf.off, vec_ok(dx, (size_t)hin * win), dxs, dx);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int launch_spec_fwd(hipStream_t st, int M, int kh, int kw, const float* filters, float* ghat) {
    return launch_rfft2<FH, FW>(st, M, kh, kw, true, filters, reinterpret_cast<cpx*>(ghat));
}

template <int FH, int FW>
int launch_spec_bwd(hipStream_t st, int M, int kh, int kw, int sh, int sw, const float* dghat,
                    float* g, int acc, int conj_in) {
    hipLaunchKernelGGL((k_filter_spectrum_bwd<FH, FW>), dim3(M), dim3(Plane<FH, FW>::NT), 0, st,
                       kh, kw, sh, sw, reinterpret_cast<const cpx*>(dghat), g, acc, conj_in);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int launch_filter_patch(hipStream_t st, int M, int kh, int kw, int sh, int sw,
                        const float* dghat, float* g, int acc, int conj_in, int hp, int wp,
                        int psh, int psw, const float* shat, const float* ghat, float* gp,
                        void* ws) {
    // the patch's cotangent spectrum (unpacked) into the workspace, then both inverses
    cpx* pspec = reinterpret_cast<cpx*>(ws);
    const int np = FH * (FW / 2);
    hipLaunchKernelGGL(k_hat_red, dim3((np + 255) / 256), dim3(256), 0, st, M, FH, FW / 2, 0,
                       reinterpret_cast<const cpx*>(shat), nullptr,
                       reinterpret_cast<const cpx*>(ghat), pspec, nullptr, 0, 0);
    NC_CHECK_LAUNCH();
    hipLaunchKernelGGL((k_filter_patch_bwd<FH, FW>), dim3(M + 1), dim3(Plane<FH, FW>::NT), 0, st,
                       M, kh, kw, sh, sw, reinterpret_cast<const cpx*>(dghat), g, acc, conj_in,
                       hp, wp, psh, psw, pspec, gp);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
size_t launch_ws(int B, int M) {
    return bwd_ws<FH, FW>(B, M);
}

#define NC_DISPATCH_FFT(FH_, FW_, CALL)                                   \
    do {                                                                  \
        if (FH_ == 16 && FW_ == 16) return CALL(16, 16);                  \
        if (FH_ == 16 && FW_ == 32) return CALL(16, 32);                  \
        if (FH_ == 16 && FW_ == 64) return CALL(16, 64);                  \
        if (FH_ == 32 && FW_ == 16) return CALL(32, 16);                  \
        if (FH_ == 32 && FW_ == 32) return CALL(32, 32);                  \
        if (FH_ == 32 && FW_ == 64) return CALL(32, 64);                  \
        if (FH_ == 64 && FW_ == 16) return CALL(64, 16);                  \
        if (FH_ == 64 && FW_ == 32) return CALL(64, 32);                  \
        if (FH_ == 64 && FW_ == 64) return CALL(64, 64);                  \
    } while (0)

}  // namespace

namespace {

// Elementwise map of nplanes (FH, FWh+1) half-spectra (FWh = FW/2): conjugate the input
// (conj_in), replace the DC and Nyquist columns by their Hermitian parts along the column
// (herm: (v[kh] + conj(v[-kh])) / 2), scale the edge columns by `edge` and the others by
// `interior`, and multiply by the phase ramp W^(kh*sh) W^(kw*sw), W = exp(-2 pi i / grid)
// (the spectrum of the plane circularly shifted by (sh, sw)).  in == NULL maps the constant
// spectrum 1.  One thread per bin.
__global__ __launch_bounds__(256) void k_spectrum_map(int nplanes, int FH, int FWh, int sh,
                                                      int sw, int herm, float edge,
                                                      float interior, int conj_in,
                                                      const cpx* in, cpx* out) {
    const int SP = FWh + 1, F = FH * SP;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)nplanes * F) return;
    const size_t p = i / F;
    const int e = (int)(i - p * F), kh = e / SP, kw = e - kh * SP;
    const bool ec = kw == 0 || kw == FWh;
    cpx v = in ? in[i] : cmk(1.0f, 0.0f);
    if (conj_in) v.y = -v.y;
    if (herm && ec && in) {
        cpx m = in[p * F + (size_t)((FH - kh) & (FH - 1)) * SP + kw];
        if (conj_in) m.y = -m.y;
        v = cmk(0.5f * (v.x + m.x), 0.5f * (v.y - m.y));
    }
    v = cscale(v, ec ? edge : interior);
    if (sh | sw) {
        // exact integer phase indices; the angles are exact binary fractions of pi
        const int a = (int)(((long long)kh * sh) & (FH - 1));
        const int b = (int)(((long long)kw * sw) & (2 * FWh - 1));
        float s1, c1, s2, c2;
        sincospif(-2.0f * (float)a / (float)FH, &s1, &c1);
        sincospif(-(float)b / (float)FWh, &s2, &c2);
        v = cmul(v, cmk(c1 * c2 - s1 * s2, s1 * c2 + c1 * s2));
    }
    out[i] = v;
}

bool any_pow2(int n) { return n >= 2 && n <= 4096 && (n & (n - 1)) == 0; }

size_t spec_bytes(int nplanes, int fh, int fw) {
    return ((size_t)nplanes * fh * (fw / 2 + 1) * sizeof(cpx) + 255) / 256 * 256;
}

}  // namespace

extern "C" {

int nc_filter_spectrum_fwd(void* stream, int M, int kh, int kw, int fft_h, int fft_w,
                           const float* filters, float* ghat) {
    if (M <= 0 || kh <= 0 || kw <= 0 || kh > fft_h || kw > fft_w || !filters || !ghat)
        return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    if (nc_large_grid(fft_h, fft_w))
        return nc_large_filter_spectrum_fwd(st, M, kh, kw, fft_h, fft_w, filters, ghat);
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return NC_ERR_UNSUPPORTED;
#define NC_CALL(A, Bv) launch_spec_fwd<A, Bv>(st, M, kh, kw, filters, ghat)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_filter_spectrum_bwd(void* stream, int M, int kh, int kw, int fft_h, int fft_w,
                           int shift_h, int shift_w, const float* dghat, float* g_filters,
                           int accumulate, int conj_in) {
    if (M <= 0 || kh <= 0 || kw <= 0 || kh > fft_h || kw > fft_w || !dghat || !g_filters ||
        shift_h < 0 || shift_w < 0)
        return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    if (nc_large_grid(fft_h, fft_w))
        return nc_large_filter_spectrum_bwd(st, M, kh, kw, fft_h, fft_w, shift_h, shift_w, dghat,
                                            g_filters, accumulate, conj_in);
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return NC_ERR_UNSUPPORTED;
#define NC_CALL(A, Bv) \
    launch_spec_bwd<A, Bv>(st, M, kh, kw, shift_h, shift_w, dghat, g_filters, accumulate, conj_in)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_filter_patch_bwd(void* stream, int M, int kh, int kw, int fft_h, int fft_w,
                        int shift_h, int shift_w, const float* dghat, float* g_filters,
                        int accumulate, int conj_in, int hp, int wp, int pshift_h, int pshift_w,
                        const float* gz_hat, const float* ghat, float* g_patch, void* ws,
                        size_t ws_bytes) {
    if (M <= 0 || kh <= 0 || kw <= 0 || kh > fft_h || kw > fft_w || !dghat || !g_filters ||
        shift_h < 0 || shift_w < 0 || hp <= 0 || wp <= 0 || hp > fft_h || wp > fft_w ||
        pshift_h < 0 || pshift_w < 0 || !gz_hat || !ghat || !g_patch)
        return NC_ERR_INVALID_ARGUMENT;
    if (nc_large_grid(fft_h, fft_w) || !pow2_ok(fft_h) || !pow2_ok(fft_w)) {
        // the workgroup-segment grids: the two operations one after the other
        const int rc = nc_filter_spectrum_bwd(stream, M, kh, kw, fft_h, fft_w, shift_h, shift_w,
                                              dghat, g_filters, accumulate, conj_in);
        if (rc != NC_OK) return rc;
        return nc_fftconv_bwd_hat(stream, M, hp, wp, pshift_h, pshift_w, fft_h, fft_w, gz_hat,
                                  nullptr, ghat, g_patch, nullptr, 0, 0, ws, ws_bytes);
    }
    if (ws_bytes < (size_t)fft_h * (fft_w / 2 + 1) * sizeof(cpx) || !ws) return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
#define NC_CALL(A, Bv)                                                                       \
    launch_filter_patch<A, Bv>(st, M, kh, kw, shift_h, shift_w, dghat, g_filters, accumulate, \
                               conj_in, hp, wp, pshift_h, pshift_w, gz_hat, ghat, g_patch, ws)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

static int fftconv_check(int B, int M, int hin, int win, int hout, int wout, int ph, int pw,
                         int fh, int fw) {
    if (B <= 0 || M <= 0 || hin <= 0 || win <= 0 || hout <= 0 || wout <= 0 || ph < 0 ||
        pw < 0)
        return NC_ERR_INVALID_ARGUMENT;
    if (!(pow2_ok(fh) && pow2_ok(fw)) && !nc_large_grid(fh, fw)) return NC_ERR_UNSUPPORTED;
    // the output window is read modulo the grid: a circular correlation where it wraps
    if (hin > fh || win > fw || hout > fh || wout > fw || ph >= fh || pw >= fw)
        return NC_ERR_INVALID_ARGUMENT;
    return NC_OK;
}

int nc_fftconv_fwd_parts(void* stream, int B, int M, int hin, int win, int hout, int wout,
                         int pad_h, int pad_w, int fft_h, int fft_w, const float* x_parts,
                         int n_parts, const float* xhat_add, const float* ghat, float* z,
                         float* xhat) {
    int rc = fftconv_check(B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (!x_parts || n_parts <= 0 || !ghat || !z || !xhat) return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    if (nc_large_grid(fft_h, fft_w))
        return nc_large_fftconv_fwd(st, B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w,
                                    x_parts, n_parts, xhat_add, ghat, z, xhat);
#define NC_CALL(A, Bv)                                                                      \
    launch_fwd<A, Bv>(st, B, M, hin, win, hout, wout, pad_h, pad_w, x_parts, n_parts, xhat_add, \
                      ghat, z, xhat)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_fftconv_fwd_ex(void* stream, int B, int M, int hin, int win, int hout, int wout,
                      int pad_h, int pad_w, int fft_h, int fft_w, const float* x,
                      const float* xhat_add, const float* ghat, float* z, float* xhat) {
    return nc_fftconv_fwd_parts(stream, B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w,
                                x, 1, xhat_add, ghat, z, xhat);
}

int nc_fftconv_fwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int pad_h,
                   int pad_w, int fft_h, int fft_w, const float* x, const float* ghat, float* z,
                   float* xhat) {
    return nc_fftconv_fwd_ex(stream, B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w, x,
                             nullptr, ghat, z, xhat);
}

int nc_plane_spectrum(void* stream, int nplanes, int hin, int win, int fft_h, int fft_w,
                      int shift_h, int shift_w, const float* x, float* xhat) {
    if (nplanes <= 0 || hin <= 0 || win <= 0 || hin > fft_h || win > fft_w || shift_h < 0 ||
        shift_w < 0 || shift_h >= fft_h || shift_w >= fft_w || !x || !xhat)
        return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    if (nc_large_grid(fft_h, fft_w))
        return nc_large_plane_spectrum(st, nplanes, hin, win, fft_h, fft_w, shift_h, shift_w, x,
                                       xhat);
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return NC_ERR_UNSUPPORTED;
    const SpecPost post{nullptr, shift_h, shift_w};
#define NC_CALL(A, Bv)                                                                   \
    launch_rfft2<A, Bv>(st, nplanes, hin, win, false, x, reinterpret_cast<cpx*>(xhat), \
                        kPostShift, post)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_plane_spectra(void* stream, int fft_h, int fft_w, int n_jobs, const nc_spectrum_job* jobs) {
    if (n_jobs <= 0 || n_jobs > kMaxSpecJobs || !jobs) return NC_ERR_INVALID_ARGUMENT;
    for (int q = 0; q < n_jobs; ++q) {
        const nc_spectrum_job& j = jobs[q];
        const int ops = (j.flip != 0) + (j.add != nullptr) + ((j.shift_h | j.shift_w) != 0);
        if (!j.x || !j.xhat || j.nplanes <= 0 || j.hin <= 0 || j.win <= 0 || j.hin > fft_h ||
            j.win > fft_w || j.shift_h < 0 || j.shift_w < 0 || j.shift_h >= fft_h ||
            j.shift_w >= fft_w || ops > 1)
            return NC_ERR_INVALID_ARGUMENT;
    }
    hipStream_t st = nc_stream(stream);
    if (nc_large_grid(fft_h, fft_w))
        return nc_large_plane_spectra(st, fft_h, fft_w, n_jobs, jobs);
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return NC_ERR_UNSUPPORTED;
#define NC_CALL(A, Bv) launch_spectra<A, Bv>(st, n_jobs, jobs)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_spectral_correlate(void* stream, int B, int M, int hout, int wout, int pad_h, int pad_w,
                          int fft_h, int fft_w, const float* xhat, const float* ghat, float* z) {
    int rc = fftconv_check(B, M, 1, 1, hout, wout, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (!xhat || !ghat || !z) return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    if (nc_large_grid(fft_h, fft_w))
        return nc_large_correlate(st, B, M, hout, wout, pad_h, pad_w, fft_h, fft_w, xhat, ghat, z);
#define NC_CALL(A, Bv) launch_corr<A, Bv>(st, B, M, hout, wout, pad_h, pad_w, xhat, ghat, z)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_fftconv_spectra(void* stream, int B, int hin, int win, int fft_h, int fft_w,
                       const float* x_parts, int n_parts, const float* xhat_add, float* xhat) {
    if (B <= 0 || hin <= 0 || win <= 0 || hin > fft_h || win > fft_w || !x_parts ||
        n_parts <= 0 || !xhat)
        return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    const size_t qs = (size_t)B * hin * win;
    if (nc_large_grid(fft_h, fft_w))
        return nc_seg_rfft2(st, fft_h, fft_w, B, hin, win, 0, x_parts, xhat, xhat_add, 0, 0,
                            n_parts, qs);
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return NC_ERR_UNSUPPORTED;
    const SpecPost post{reinterpret_cast<const cpx*>(xhat_add), 0, 0};
#define NC_CALL(A, Bv)                                                                   \
    launch_rfft2<A, Bv>(st, B, hin, win, false, x_parts, reinterpret_cast<cpx*>(xhat), \
                        xhat_add ? kPostAdd : kPostNone, post, n_parts, qs)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

size_t nc_fftconv_correlate_workspace_size(int B, int M, int hout, int wout, int fft_h,
                                           int fft_w) {
    if (B <= 0 || M <= 0 || hout <= 0 || wout <= 0 || !nc_large_grid(fft_h, fft_w)) return 0;
    return nc_large_correlate_ws(B, M, hout, fft_h, fft_w);
}

}  // extern "C"

namespace {
// nc_spectral_correlate, by the two-pass large-grid transform when ws holds its intermediate.
int correlate_ws(void* stream, int B, int M, int hout, int wout, int pad_h, int pad_w, int fft_h,
                 int fft_w, const float* xhat, const float* ghat, float* z, void* ws,
                 size_t ws_bytes) {
    if (ws && nc_large_grid(fft_h, fft_w) &&
        ws_bytes >= nc_fftconv_correlate_workspace_size(B, M, hout, wout, fft_h, fft_w)) {
        int rc = fftconv_check(B, M, 1, 1, hout, wout, pad_h, pad_w, fft_h, fft_w);
        if (rc != NC_OK) return rc;
        if (!xhat || !ghat || !z) return NC_ERR_INVALID_ARGUMENT;
        return nc_large_correlate(nc_stream(stream), B, M, hout, wout, pad_h, pad_w, fft_h, fft_w,
                                  xhat, ghat, z, ws, ws_bytes);
    }
    return nc_spectral_correlate(stream, B, M, hout, wout, pad_h, pad_w, fft_h, fft_w, xhat, ghat,
                                 z);
}
}  // namespace

extern "C" {

size_t nc_fftconv_port_workspace_size(int B, int M, int h, int w, int fft_h, int fft_w,
                                      int n_port) {
    const size_t epi = nc_epilogue_workspace_size(B, M, h, w);
    if (B <= 0 || M <= 0 || n_port <= 0 || corr_epi_region(fft_h, fft_w, h, w) == 0) return epi;
    return std::max(epi, (size_t)2 * ((M + 3) / 4) * B * n_port * sizeof(float));
}

int nc_fftconv_port_fwd(void* stream, int B, int M, int hout, int wout, int pad_h, int pad_w,
                        int fft_h, int fft_w, const float* xhat, const float* ghat,
                        int final_act, float neg_slope, int n_port, const int32_t* port_idx,
                        const float* port_params, float* z, float* out, float* zo, float* mean,
                        float* rstd, float* pre, void* ws, size_t ws_bytes) {
    int rc = fftconv_check(B, M, 1, 1, hout, wout, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (!xhat || !ghat || n_port <= 0 || n_port > 256 || M * n_port > 8192 || !port_idx ||
        !port_params || !out || !zo || !mean || !rstd || final_act < 0 || final_act > 5 ||
        (final_act != NC_ACT_IDENTITY && !pre))
        return NC_ERR_INVALID_ARGUMENT;
    if (ws_bytes < nc_fftconv_port_workspace_size(B, M, hout, wout, fft_h, fft_w, n_port) || !ws)
        return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
    float* part = reinterpret_cast<float*>(ws);
    bool done = false;
    if (corr_epi_region(fft_h, fft_w, hout, wout) > 0) {
        if (fft_h == 64)
            done = launch_corr_port<64, 64>(st, B, M, hout, wout, pad_h, pad_w, n_port,
                                            final_act, neg_slope, xhat, ghat, port_idx,
                                            port_params, z, zo, mean, rstd, part);
        else
            done = launch_corr_port<32, 64>(st, B, M, hout, wout, pad_h, pad_w, n_port,
                                            final_act, neg_slope, xhat, ghat, port_idx,
                                            port_params, z, zo, mean, rstd, part);
    }
    if (done) {
        NC_CHECK_LAUNCH();
        return nc_port_combine_launch(st, B, M, n_port, (M + 3) / 4, final_act, neg_slope,
                                      port_params, part, out, pre);
    }
    // other grids: the correlation into z (two-pass through ws when it is large enough), then
    // the port
    if (!z) return NC_ERR_INVALID_ARGUMENT;
    rc = correlate_ws(stream, B, M, hout, wout, pad_h, pad_w, fft_h, fft_w, xhat, ghat, z, ws,
                      ws_bytes);
    if (rc != NC_OK) return rc;
    return nc_port_fwd(stream, B, M, hout, wout, 0, final_act, neg_slope, n_port, port_idx, z,
                       nullptr, port_params, out, zo, mean, rstd, pre, ws, ws_bytes);
}

int nc_fftconv_epilogue_partials(int B, int M, int h, int w, int fft_h, int fft_w) {
    if (B <= 0 || M <= 0 || h <= 0 || w <= 0) return 0;
    if (corr_epi_region(fft_h, fft_w, h, w) > 0) return (M + 3) / 4;
    return nc_epilogue_fwd_partials(B, M, h, w);
}

int nc_fftconv_epilogue_fwd(void* stream, int B, int M, int hout, int wout, int pad_h,
                            int pad_w, int fft_h, int fft_w, const float* xhat,
                            const float* ghat, int act, float neg_slope, const float* w_eff,
                            const float* s_eff, const float* b_roi, float* z, float* parts,
                            float* mean, float* rstd, void* ws, size_t ws_bytes) {
    int rc = fftconv_check(B, M, 1, 1, hout, wout, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (!xhat || !ghat || !w_eff || !s_eff || !b_roi || !parts || !mean || !rstd || act < 0 ||
        act > 5)
        return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    bool done = false;
    if (corr_epi_region(fft_h, fft_w, hout, wout) > 0) {
        if (fft_h == 64)
            done = launch_corr_epi<64, 64>(st, B, M, hout, wout, pad_h, pad_w, act, neg_slope,
                                           xhat, ghat, w_eff, s_eff, b_roi, z, parts, mean,
                                           rstd);
        else
            done = launch_corr_epi<32, 64>(st, B, M, hout, wout, pad_h, pad_w, act, neg_slope,
                                           xhat, ghat, w_eff, s_eff, b_roi, z, parts, mean,
                                           rstd);
        if (done) {
            NC_CHECK_LAUNCH();
            return NC_OK;
        }
    }
    // other grids: the correlation into z (two-pass through ws when it is large enough), then
    // the epilogue's partial outputs
    if (!z) return NC_ERR_INVALID_ARGUMENT;
    if (nc_large_grid(fft_h, fft_w) && nc_epilogue_tiled(hout * wout) && ws &&
        ws_bytes >= nc_fftconv_correlate_workspace_size(B, M, hout, wout, fft_h, fft_w) &&
        (size_t)B * M <= 65535) {
        // the two-pass correlation's row pass also forms the tiled epilogue's statistics, per
        // band of rows (kept in ws past the intermediate), so z is read once more, not twice
        const int br = nc_large_band_rows(fft_h, fft_w);
        float* stats = reinterpret_cast<float*>(
            static_cast<char*>(ws) + nc_large_band_stats_offset(B, M, hout, fft_h, fft_w));
        rc = nc_large_correlate(st, B, M, hout, wout, pad_h, pad_w, fft_h, fft_w, xhat, ghat, z,
                                ws, ws_bytes, stats);
        if (rc != NC_OK) return rc;
        return nc_epilogue_fwd_from_stats(st, B, M, hout, wout, act, neg_slope, z, w_eff, s_eff,
                                          b_roi, stats, (hout + br - 1) / br, br * wout, parts,
                                          mean, rstd);
    }
    rc = correlate_ws(stream, B, M, hout, wout, pad_h, pad_w, fft_h, fft_w, xhat, ghat, z, ws,
                      ws_bytes);
    if (rc != NC_OK) return rc;
    return nc_epilogue_fwd_parts(stream, B, M, hout, wout, act, neg_slope, 0, z, nullptr, w_eff,
                                 s_eff, b_roi, parts, mean, rstd, ws, ws_bytes);
}

size_t nc_fftconv_bwd_workspace_size(int B, int M, int fft_h, int fft_w) {
    if (B <= 0 || M <= 0) return 0;
    if (nc_large_grid(fft_h, fft_w)) return nc_large_fftconv_bwd_ws(B, M, fft_h, fft_w);
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return 0;
#define NC_CALL(A, Bv) launch_ws<A, Bv>(B, M)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return 0;
}

static int fftconv_bwd(void* stream, int B, int M, int hin, int win, int hout, int wout,
                       int pad_h, int pad_w, int fft_h, int fft_w, const float* gz,
                       const float* xhat, const float* ghat, int need_dx, float* dx, float* dghat,
                       int accumulate, int conj_dghat, float* gz_hat_sum, int sum_accumulate,
                       bool parts, void* ws, size_t ws_bytes) {
    int rc = fftconv_check(B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (!gz || !xhat || !ghat || !dghat || (need_dx && !dx)) return NC_ERR_INVALID_ARGUMENT;
    if (ws_bytes < nc_fftconv_bwd_workspace_size(B, M, fft_h, fft_w) || !ws)
        return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
    if (nc_large_grid(fft_h, fft_w))
        return nc_large_fftconv_bwd(st, B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w,
                                    gz, xhat, ghat, need_dx, dx, dghat, accumulate, conj_dghat,
                                    gz_hat_sum, sum_accumulate, parts ? 1 : 0, ws);
#define NC_CALL(A, Bv)                                                                     \
    launch_bwd<A, Bv>(st, B, M, hin, win, hout, wout, pad_h, pad_w, gz, xhat, ghat, need_dx, \
                      dx, dghat, accumulate, conj_dghat, gz_hat_sum, sum_accumulate, parts, ws)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_fftconv_bwd_ex(void* stream, int B, int M, int hin, int win, int hout, int wout,
                      int pad_h, int pad_w, int fft_h, int fft_w, const float* gz,
                      const float* xhat, const float* ghat, int need_dx, float* dx, float* dghat,
                      int accumulate, int conj_dghat, float* gz_hat_sum, int sum_accumulate,
                      void* ws, size_t ws_bytes) {
    return fftconv_bwd(stream, B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w, gz, xhat,
                       ghat, need_dx, dx, dghat, accumulate, conj_dghat, gz_hat_sum,
                       sum_accumulate, false, ws, ws_bytes);
}

int nc_fftconv_bwd_partials(int B, int M, int fft_h, int fft_w) {
    if (B <= 0 || M <= 0) return 0;
    if (nc_large_grid(fft_h, fft_w)) return nc_large_red_splits(B, M, fft_h, fft_w);
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return 0;
#define NC_CALL(A, Bv) dg_parts<A, Bv>(B, M)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return 0;
}

int nc_fftconv_bwd_parts(void* stream, int B, int M, int hin, int win, int hout, int wout,
                         int pad_h, int pad_w, int fft_h, int fft_w, const float* gz,
                         const float* xhat, const float* ghat, int need_dx, float* dx,
                         float* dghat_parts, int accumulate, int conj_dghat,
                         float* gz_hat_sum_parts, int sum_accumulate, void* ws, size_t ws_bytes) {
    return fftconv_bwd(stream, B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w, gz, xhat,
                       ghat, need_dx, dx, dghat_parts, accumulate, conj_dghat, gz_hat_sum_parts,
                       sum_accumulate, true, ws, ws_bytes);
}

int nc_epilogue_fftconv_bwd_parts(void* stream, int B, int M, int h, int w, int act,
                                  float neg_slope, const float* z, const float* w_eff,
                                  const float* s_eff, const float* b_roi, const float* mean,
                                  const float* rstd, const float* gy, float* gz, float* pg_rows,
                                  size_t plane_stride, int hin, int win, int pad_h, int pad_w,
                                  int fft_h, int fft_w, const float* xhat, const float* ghat,
                                  int need_dx, float* dx, float* dghat_parts, int accumulate,
                                  int conj_dghat, float* gz_hat_sum_parts, int sum_accumulate,
                                  void* ws_epi, size_t ws_epi_bytes, void* ws_fc,
                                  size_t ws_fc_bytes) {
    int rc = fftconv_check(B, M, hin, win, h, w, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (nc_large_grid(fft_h, fft_w) && nc_epilogue_tiled(h * w) && (size_t)B * M <= 65535) {
        // the cotangent spectra's row pass forms gz from the epilogue's inputs: gz is neither
        // stored nor read back
        if (!xhat || !ghat || !dghat_parts || (need_dx && !dx)) return NC_ERR_INVALID_ARGUMENT;
        if (ws_fc_bytes < nc_fftconv_bwd_workspace_size(B, M, fft_h, fft_w) || !ws_fc)
            return NC_ERR_WORKSPACE;
        hipStream_t st = nc_stream(stream);
        nc_epi_gz e{z, w_eff, s_eff, b_roi, gy, mean, rstd, nullptr, 0, act, neg_slope};
        rc = nc_epilogue_bwd_stage1(st, B, M, h, w, act, neg_slope, z, w_eff, s_eff, b_roi, mean,
                                    rstd, gy, pg_rows, plane_stride, ws_epi, ws_epi_bytes,
                                    &e.cpart, &e.n_tiles);
        if (rc != NC_OK) return rc;
        return nc_large_fftconv_bwd_epi(st, B, M, hin, win, h, w, pad_h, pad_w, fft_h, fft_w, e,
                                        xhat, ghat, need_dx, dx, dghat_parts, accumulate,
                                        conj_dghat, gz_hat_sum_parts, sum_accumulate, 1, ws_fc);
    }
    rc = nc_epilogue_bwd_parts(stream, B, M, h, w, act, neg_slope, 0, z, nullptr, w_eff, s_eff,
                               b_roi, mean, rstd, gy, gz, pg_rows, plane_stride, ws_epi,
                               ws_epi_bytes);
    if (rc != NC_OK) return rc;
    return nc_fftconv_bwd_parts(stream, B, M, hin, win, h, w, pad_h, pad_w, fft_h, fft_w, gz,
                                xhat, ghat, need_dx, dx, dghat_parts, accumulate, conj_dghat,
                                gz_hat_sum_parts, sum_accumulate, ws_fc, ws_fc_bytes);
}

int nc_fftconv_bwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int pad_h,
                   int pad_w, int fft_h, int fft_w, const float* gz, const float* xhat,
                   const float* ghat, int need_dx, float* dx, float* dghat, int accumulate,
                   int conj_dghat, void* ws, size_t ws_bytes) {
    return nc_fftconv_bwd_ex(stream, B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w, gz,
                             xhat, ghat, need_dx, dx, dghat, accumulate, conj_dghat, nullptr, 0,
                             ws, ws_bytes);
}

int nc_fftconv_bwd_hat(void* stream, int M, int hin, int win, int pad_h, int pad_w, int fft_h,
                       int fft_w, const float* gz_hat, const float* xhat, const float* ghat,
                       float* dx, float* dghat, int accumulate, int conj_dghat, void* ws,
                       size_t ws_bytes) {
    if (M <= 0 || hin <= 0 || win <= 0 || pad_h < 0 || pad_w < 0 || hin > fft_h ||
        win > fft_w || !gz_hat || !ghat || !dx || (dghat && !xhat))
        return NC_ERR_INVALID_ARGUMENT;
    if (!(pow2_ok(fft_h) && pow2_ok(fft_w)) && !nc_large_grid(fft_h, fft_w))
        return NC_ERR_UNSUPPORTED;
    const size_t F = (size_t)fft_h * (fft_w / 2 + 1);
    if (ws_bytes < F * sizeof(cpx) || !ws) return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
    const bool large = nc_large_grid(fft_h, fft_w);
    const bool packed = !large && !(fft_w == 64 && (fft_h == 32 || fft_h == 64));
    cpx* dxs = reinterpret_cast<cpx*>(ws);
    const int np = fft_h * (fft_w / 2);
    hipLaunchKernelGGL(k_hat_red, dim3((np + 255) / 256), dim3(256), 0, st, M, fft_h, fft_w / 2,
                       packed ? 1 : 0, reinterpret_cast<const cpx*>(gz_hat),
                       reinterpret_cast<const cpx*>(xhat), reinterpret_cast<const cpx*>(ghat),
                       dxs, reinterpret_cast<cpx*>(dghat), accumulate, conj_dghat);
    NC_CHECK_LAUNCH();
    if (large) return nc_large_hat_dx(st, hin, win, pad_h, pad_w, fft_h, fft_w, dxs, dx);
#define NC_CALL(A, Bv) launch_hat_dx<A, Bv>(st, hin, win, pad_h, pad_w, dxs, dx)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
    return NC_ERR_UNSUPPORTED;
}

int nc_spectrum_map(void* stream, int nplanes, int fft_h, int fft_w, int shift_h, int shift_w,
                    int herm_edges, float edge_scale, float interior_scale, int conj_in,
                    const float* in, float* out) {
    if (nplanes <= 0 || !any_pow2(fft_h) || !any_pow2(fft_w) || shift_h < 0 || shift_w < 0 ||
        shift_h >= fft_h || shift_w >= fft_w || !out || (herm_edges && in == out))
        return NC_ERR_INVALID_ARGUMENT;
    const size_t n = (size_t)nplanes * fft_h * (fft_w / 2 + 1);
    hipLaunchKernelGGL(k_spectrum_map, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       nc_stream(stream), nplanes, fft_h, fft_w / 2, shift_h, shift_w,
                       herm_edges, edge_scale, interior_scale, conj_in,
                       reinterpret_cast<const cpx*>(in), reinterpret_cast<cpx*>(out));
    NC_CHECK_LAUNCH();
    return NC_OK;
}

size_t nc_irfft2_pruned_workspace_size(int nplanes, int fft_h, int fft_w) {
    if (nplanes <= 0 || fft_h <= 0 || fft_w <= 0) return 0;
    return spec_bytes(nplanes, fft_h, fft_w) + spec_bytes(1, fft_h, fft_w);
}

int nc_irfft2_pruned(void* stream, int nplanes, int hout, int wout, int pad_h, int pad_w,
                     int fft_h, int fft_w, const float* xhat, float* out, void* ws,
                     size_t ws_bytes) {
    int rc = fftconv_check(nplanes, 1, 1, 1, hout, wout, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (!xhat || !out) return NC_ERR_INVALID_ARGUMENT;
    if (!ws || ws_bytes < nc_irfft2_pruned_workspace_size(nplanes, fft_h, fft_w))
        return NC_ERR_WORKSPACE;
    // the Hermitian parts of the edge columns (what a real inverse keeps of them), then the
    // correlation of those spectra with the constant spectrum 1 over the output window
    float* proj = reinterpret_cast<float*>(ws);
    float* ones = reinterpret_cast<float*>(static_cast<char*>(ws) +
                                           spec_bytes(nplanes, fft_h, fft_w));
    rc = nc_spectrum_map(stream, nplanes, fft_h, fft_w, 0, 0, 1, 1.0f, 1.0f, 0, xhat, proj);
    if (rc != NC_OK) return rc;
    rc = nc_spectrum_map(stream, 1, fft_h, fft_w, 0, 0, 0, 1.0f, 1.0f, 0, nullptr, ones);
    if (rc != NC_OK) return rc;
    return nc_spectral_correlate(stream, nplanes, 1, hout, wout, pad_h, pad_w, fft_h, fft_w,
                                 proj, ones, out);
}

}  // extern "C"

// Piece 2: Green's-function convolution as LDS-resident, row-pruned overlap-save rfft2.
//
// Kernels (one (FH x FW) plane per workgroup step, FH, FW in {16, 32, 64}):
//   k_filter_spectrum_fwd  grid (M)           ghat_m = rfft2(flip(G_m))
//   k_filter_spectrum_bwd  grid (M)           dG_m = flip(crop(roll(irfft2(dghat_m))))
//   k_fftconv_fwd          grid (B, M/MC)     xhat_b once per workgroup, then for each m:
//                                             z_bm = irfft2(xhat_b * ghat_m) (cropped window)
//   k_fftconv_bwd_dx       grid (B, MS)       A_b = sum_m rfft2(gz_bm) * conj(ghat_m) over an
//                                             M-split; with MS == 1 the inverse runs in place
//   k_fftconv_bwd_dx_fin   grid (B)           sums the MS partial spectra (fixed order), irfft2
//   k_fftconv_bwd_dg       grid (M, NBC)      D_m = sum_b rfft2(gz_bm) * conj(xhat_b) over a
//                                             B-chunk (kept in registers)
//   k_fftconv_bwd_dg_fin   grid (M, F/256)    sums the NBC chunk partials in fixed order
// No atomics anywhere: the M- and B-reductions are two-stage trees in the frequency domain.
#include <algorithm>

#include "nc_fft.h"

namespace {

template <int FH, int FW>
struct Smem {
    using P = Plane<FH, FW>;
    cpx work[P::WORK];
    cpx scr[P::SCRN];
    cpx tw[NC_TW_N];
};

// Every kernel starts by copying the twiddle table into LDS.
#define NC_SPECTRAL_PROLOGUE(sm) \
    load_twiddles(sm.tw);        \
    __syncthreads()

// ----------------------------------------------------------------------------------------
// Filter spectrum (kernels_greens.py:240-259) and its backward (kernels_pallas.py:1558-1579)
// ----------------------------------------------------------------------------------------

template <int FH, int FW>
__global__ __launch_bounds__((Plane<FH, FW>::NT)) void k_filter_spectrum_fwd(
    int kh, int kw, const float* __restrict__ filt, cpx* __restrict__ ghat) {
    using P = Plane<FH, FW>;
    __shared__ cpx S[P::F];
    __shared__ Smem<FH, FW> sm;
    NC_SPECTRAL_PROLOGUE(sm);
    const int m = blockIdx.x;
    const float* g = filt + (size_t)m * kh * kw;
    // flipped filter: x[r][c] = G[kh-1-r][kw-1-c]
    plane_rfft2<FH, FW>([&](int r, int c) { return g[(kh - 1 - r) * kw + (kw - 1 - c)]; },
                        kh, kw, S, sm.work, sm.scr, sm.tw);
    for (int e = threadIdx.x; e < P::F; e += P::NT) ghat[(size_t)m * P::F + e] = S[e];
}

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
            cpx v = d[a * P::SP + b];
            return conj_in ? cconj(v) : v;
        },
        row0, kh, col0, kw, 1.0f / (float)(FH * FW),
        [&](int i, int j, float v) {
            float* o = out + (kh - 1 - i) * kw + (kw - 1 - j);
            *o = accumulate ? *o + v : v;
        },
        sm.work, sm.scr, sm.tw);
}

// ----------------------------------------------------------------------------------------
// Forward correlation (kernels_pallas.py:1779-1791; kernels_greens.py:316-343)
// ----------------------------------------------------------------------------------------

template <int FH, int FW>
__global__ __launch_bounds__((Plane<FH, FW>::NT)) void k_fftconv_fwd(
    int M, int mc, int hin, int win, int hout, int wout, int ph, int pw,
    const float* __restrict__ x, const cpx* __restrict__ ghat, float* __restrict__ z,
    cpx* __restrict__ xhat) {
    using P = Plane<FH, FW>;
    __shared__ cpx S[P::F];
    __shared__ Smem<FH, FW> sm;
    __shared__ float O[FH * FW];
    NC_SPECTRAL_PROLOGUE(sm);
    const int b = blockIdx.x;
    const int m0 = blockIdx.y * mc;
    const int m1 = min(M, m0 + mc);
    // stage the sample's plane (coalesced) into S, which the row pass reads before the
    // column pass overwrites it with the spectrum
    float* Sf = reinterpret_cast<float*>(S);
    stage_plane(x + (size_t)b * hin * win, hin * win, Sf);
    __syncthreads();
    plane_rfft2<FH, FW>([&](int r, int c) { return Sf[r * win + c]; }, hin, win, S, sm.work,
                        sm.scr, sm.tw);
    if (xhat != nullptr && blockIdx.y == 0)
        for (int e = threadIdx.x; e < P::F; e += P::NT) xhat[(size_t)b * P::F + e] = S[e];
    const int npix = hout * wout;
    const float scale = 1.0f / (float)(FH * FW);
    for (int m = m0; m < m1; ++m) {
        const cpx* G = ghat + (size_t)m * P::F;
        plane_irfft2<FH, FW>(
            [&](int a, int c) { return cmul(S[a * P::SP + c], G[a * P::SP + c]); }, ph, hout,
            pw, wout, scale, [&](int i, int j, float v) { O[i * wout + j] = v; }, sm.work,
            sm.scr, sm.tw);
        float* zo = z + ((size_t)b * M + m) * npix;
        for (int e = threadIdx.x; e < npix; e += P::NT) zo[e] = O[e];
        // O is rewritten only after the next inverse's column phase barriers.
    }
}

// ----------------------------------------------------------------------------------------
// Backward: dx (M-reduction) and dghat (B-reduction), kernels_pallas.py:1794-1821
// ----------------------------------------------------------------------------------------

template <int FH, int FW>
__global__ __launch_bounds__((Plane<FH, FW>::NT)) void k_fftconv_bwd_dx(
    int M, int ms_size, int hin, int win, int hout, int wout, int ph, int pw,
    const float* __restrict__ gz, const cpx* __restrict__ ghat, cpx* __restrict__ part,
    float* __restrict__ dx) {
    using P = Plane<FH, FW>;
    __shared__ cpx S[P::F];
    __shared__ cpx A[P::F];
    __shared__ Smem<FH, FW> sm;
    NC_SPECTRAL_PROLOGUE(sm);
    const int b = blockIdx.x;
    const int m0 = blockIdx.y * ms_size;
    const int m1 = min(M, m0 + ms_size);
    const int npix = hout * wout;
    float* Sf = reinterpret_cast<float*>(S);
    for (int e = threadIdx.x; e < P::F; e += P::NT) A[e] = cmk(0.f, 0.f);
    for (int m = m0; m < m1; ++m) {
        stage_plane(gz + ((size_t)b * M + m) * npix, npix, Sf);
        __syncthreads();
        plane_rfft2<FH, FW>([&](int r, int c) { return Sf[r * wout + c]; }, hout, wout, S,
                            sm.work, sm.scr, sm.tw);
        const cpx* G = ghat + (size_t)m * P::F;
        for (int e = threadIdx.x; e < P::F; e += P::NT) A[e] = cadd(A[e], cmulc(S[e], G[e]));
        __syncthreads();  // S is restaged by the next direction
    }
    if (part != nullptr) {  // M split across workgroups: emit the partial spectrum
        cpx* dst = part + ((size_t)b * gridDim.y + blockIdx.y) * P::F;
        for (int e = threadIdx.x; e < P::F; e += P::NT) dst[e] = A[e];
        return;
    }
    float* d = dx + (size_t)b * hin * win;
    plane_irfft2<FH, FW>(
        [&](int a, int c) { return A[a * P::SP + c]; }, (FH - ph) & (FH - 1), hin,
        (FW - pw) & (FW - 1), win, 1.0f / (float)(FH * FW),
        [&](int i, int j, float v) { d[i * win + j] = v; }, sm.work, sm.scr, sm.tw);
}

template <int FH, int FW>
__global__ __launch_bounds__((Plane<FH, FW>::NT)) void k_fftconv_bwd_dx_fin(
    int nsplit, int hin, int win, int ph, int pw, const cpx* __restrict__ part,
    float* __restrict__ dx) {
    using P = Plane<FH, FW>;
    __shared__ cpx A[P::F];
    __shared__ Smem<FH, FW> sm;
    NC_SPECTRAL_PROLOGUE(sm);
    const int b = blockIdx.x;
    const cpx* src = part + (size_t)b * nsplit * P::F;
    for (int e = threadIdx.x; e < P::F; e += P::NT) {
        cpx s = src[e];
        for (int k = 1; k < nsplit; ++k) s = cadd(s, src[(size_t)k * P::F + e]);
        A[e] = s;
    }
    __syncthreads();
    float* d = dx + (size_t)b * hin * win;
    plane_irfft2<FH, FW>(
        [&](int a, int c) { return A[a * P::SP + c]; }, (FH - ph) & (FH - 1), hin,
        (FW - pw) & (FW - 1), win, 1.0f / (float)(FH * FW),
        [&](int i, int j, float v) { d[i * win + j] = v; }, sm.work, sm.scr, sm.tw);
}

template <int FH, int FW>
__global__ __launch_bounds__((Plane<FH, FW>::NT)) void k_fftconv_bwd_dg(
    int B, int M, int bc, int hout, int wout, const float* __restrict__ gz,
    const cpx* __restrict__ xhat, cpx* __restrict__ part) {
    using P = Plane<FH, FW>;
    constexpr int PER = (P::F + P::NT - 1) / P::NT;
    __shared__ cpx S[P::F];
    __shared__ Smem<FH, FW> sm;
    NC_SPECTRAL_PROLOGUE(sm);
    const int m = blockIdx.x;
    const int b0 = blockIdx.y * bc;
    const int b1 = min(B, b0 + bc);
    const int npix = hout * wout;
    float* Sf = reinterpret_cast<float*>(S);
    cpx acc[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) acc[u] = cmk(0.f, 0.f);
    for (int b = b0; b < b1; ++b) {
        stage_plane(gz + ((size_t)b * M + m) * npix, npix, Sf);
        __syncthreads();
        plane_rfft2<FH, FW>([&](int r, int c) { return Sf[r * wout + c]; }, hout, wout, S,
                            sm.work, sm.scr, sm.tw);
        const cpx* X = xhat + (size_t)b * P::F;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int e = threadIdx.x + u * P::NT;
            if (e < P::F) acc[u] = cadd(acc[u], cmulc(S[e], X[e]));
        }
        __syncthreads();  // S is restaged by the next sample
    }
    cpx* dst = part + ((size_t)blockIdx.y * M + m) * P::F;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int e = threadIdx.x + u * P::NT;
        if (e < P::F) dst[e] = acc[u];
    }
}

__global__ void k_fftconv_bwd_dg_fin(int nchunk, int M, int F, const cpx* __restrict__ part,
                                     cpx* __restrict__ dghat, int accumulate, int conj_out) {
    const int m = blockIdx.x;
    const int e = blockIdx.y * blockDim.x + threadIdx.x;
    if (e >= F) return;
    cpx s = part[(size_t)m * F + e];
    for (int k = 1; k < nchunk; ++k) s = cadd(s, part[((size_t)k * M + m) * F + e]);
    if (conj_out) s = cconj(s);
    cpx* o = dghat + (size_t)m * F + e;
    *o = accumulate ? cadd(*o, s) : s;
}

// ----------------------------------------------------------------------------------------
// Launch plumbing
// ----------------------------------------------------------------------------------------

bool pow2_ok(int f) { return f == 16 || f == 32 || f == 64; }

struct BwdSplit {
    int ms;      // directions per dx workgroup
    int nsplit;  // dx workgroups per sample
    int bc;      // samples per dg workgroup
    int nchunk;  // dg chunks
};

BwdSplit bwd_split(int B, int M) {
    BwdSplit s;
    int target = std::max(1, 512 / std::max(1, B));
    s.nsplit = std::min(M, target);
    s.ms = (M + s.nsplit - 1) / s.nsplit;
    s.nsplit = (M + s.ms - 1) / s.ms;
    int chunks = std::max(1, std::min(B, 256 / std::max(1, M)));
    s.bc = (B + chunks - 1) / chunks;
    s.nchunk = (B + s.bc - 1) / s.bc;
    return s;
}

template <int FH, int FW>
int launch_fwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout, int ph,
               int pw, const float* x, const float* ghat, float* z, float* xhat) {
    using P = Plane<FH, FW>;
    int mc = B >= 512 ? M : std::max(1, std::min(M, (M * B + 511) / 512));
    mc = std::max(1, std::min(M, mc));
    dim3 grid(B, (M + mc - 1) / mc);
    hipLaunchKernelGGL((k_fftconv_fwd<FH, FW>), grid, dim3(P::NT), 0, st, M, mc, hin, win,
                       hout, wout, ph, pw, x, reinterpret_cast<const cpx*>(ghat), z,
                       reinterpret_cast<cpx*>(xhat));
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int launch_bwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout, int ph,
               int pw, const float* gz, const float* xhat, const float* ghat, int need_dx,
               float* dx, float* dghat, int accumulate, int conj_out, void* ws) {
    using P = Plane<FH, FW>;
    BwdSplit s = bwd_split(B, M);
    cpx* dxpart = reinterpret_cast<cpx*>(ws);
    cpx* dgpart = dxpart + (size_t)B * s.nsplit * P::F;
    const cpx* G = reinterpret_cast<const cpx*>(ghat);
    if (need_dx) {
        hipLaunchKernelGGL((k_fftconv_bwd_dx<FH, FW>), dim3(B, s.nsplit), dim3(P::NT), 0, st,
                           M, s.ms, hin, win, hout, wout, ph, pw, gz, G,
                           s.nsplit > 1 ? dxpart : nullptr, dx);
        NC_CHECK_LAUNCH();
        if (s.nsplit > 1) {
            hipLaunchKernelGGL((k_fftconv_bwd_dx_fin<FH, FW>), dim3(B), dim3(P::NT), 0, st,
                               s.nsplit, hin, win, ph, pw, dxpart, dx);
            NC_CHECK_LAUNCH();
        }
    }
    hipLaunchKernelGGL((k_fftconv_bwd_dg<FH, FW>), dim3(M, s.nchunk), dim3(P::NT), 0, st, B, M,
                       s.bc, hout, wout, gz, reinterpret_cast<const cpx*>(xhat), dgpart);
    NC_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_fftconv_bwd_dg_fin, dim3(M, (P::F + 255) / 256), dim3(256), 0, st,
                       s.nchunk, M, P::F, dgpart, reinterpret_cast<cpx*>(dghat), accumulate,
                       conj_out);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int launch_spec_fwd(hipStream_t st, int M, int kh, int kw, const float* filters, float* ghat) {
    hipLaunchKernelGGL((k_filter_spectrum_fwd<FH, FW>), dim3(M), dim3(Plane<FH, FW>::NT), 0, st,
                       kh, kw, filters, reinterpret_cast<cpx*>(ghat));
    NC_CHECK_LAUNCH();
    return NC_OK;
}

template <int FH, int FW>
int launch_spec_bwd(hipStream_t st, int M, int kh, int kw, int sh, int sw, const float* dghat,
                    float* g, int acc, int conj_in) {
    hipLaunchKernelGGL((k_filter_spectrum_bwd<FH, FW>), dim3(M), dim3(Plane<FH, FW>::NT), 0, st,
                       kh, kw, sh, sw, reinterpret_cast<const cpx*>(dghat), g, acc, conj_in);
    NC_CHECK_LAUNCH();
    return NC_OK;
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
        return NC_ERR_UNSUPPORTED;                                        \
    } while (0)

}  // namespace

extern "C" {

int nc_filter_spectrum_fwd(void* stream, int M, int kh, int kw, int fft_h, int fft_w,
                           const float* filters, float* ghat) {
    if (M <= 0 || kh <= 0 || kw <= 0 || kh > fft_h || kw > fft_w || !filters || !ghat)
        return NC_ERR_INVALID_ARGUMENT;
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return NC_ERR_UNSUPPORTED;
    hipStream_t st = nc_stream(stream);
#define NC_CALL(A, Bv) launch_spec_fwd<A, Bv>(st, M, kh, kw, filters, ghat)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
}

int nc_filter_spectrum_bwd(void* stream, int M, int kh, int kw, int fft_h, int fft_w,
                           int shift_h, int shift_w, const float* dghat, float* g_filters,
                           int accumulate, int conj_in) {
    if (M <= 0 || kh <= 0 || kw <= 0 || kh > fft_h || kw > fft_w || !dghat || !g_filters ||
        shift_h < 0 || shift_w < 0)
        return NC_ERR_INVALID_ARGUMENT;
    if (!pow2_ok(fft_h) || !pow2_ok(fft_w)) return NC_ERR_UNSUPPORTED;
    hipStream_t st = nc_stream(stream);
#define NC_CALL(A, Bv) \
    launch_spec_bwd<A, Bv>(st, M, kh, kw, shift_h, shift_w, dghat, g_filters, accumulate, conj_in)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
}

static int fftconv_check(int B, int M, int hin, int win, int hout, int wout, int ph, int pw,
                         int fh, int fw) {
    if (B <= 0 || M <= 0 || hin <= 0 || win <= 0 || hout <= 0 || wout <= 0 || ph < 0 ||
        pw < 0)
        return NC_ERR_INVALID_ARGUMENT;
    if (!pow2_ok(fh) || !pow2_ok(fw)) return NC_ERR_UNSUPPORTED;
    if (hin > fh || win > fw || ph + hout > fh || pw + wout > fw) return NC_ERR_INVALID_ARGUMENT;
    return NC_OK;
}

int nc_fftconv_fwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int pad_h,
                   int pad_w, int fft_h, int fft_w, const float* x, const float* ghat, float* z,
                   float* xhat) {
    int rc = fftconv_check(B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (!x || !ghat || !z) return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
#define NC_CALL(A, Bv) \
    launch_fwd<A, Bv>(st, B, M, hin, win, hout, wout, pad_h, pad_w, x, ghat, z, xhat)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
}

size_t nc_fftconv_bwd_workspace_size(int B, int M, int fft_h, int fft_w) {
    if (B <= 0 || M <= 0 || fft_h <= 0 || fft_w <= 0) return 0;
    BwdSplit s = bwd_split(B, M);
    size_t F = (size_t)fft_h * (fft_w / 2 + 1);
    return ((size_t)B * s.nsplit + (size_t)s.nchunk * M) * F * sizeof(float2);
}

int nc_fftconv_bwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int pad_h,
                   int pad_w, int fft_h, int fft_w, const float* gz, const float* xhat,
                   const float* ghat, int need_dx, float* dx, float* dghat, int accumulate,
                   int conj_dghat, void* ws, size_t ws_bytes) {
    int rc = fftconv_check(B, M, hin, win, hout, wout, pad_h, pad_w, fft_h, fft_w);
    if (rc != NC_OK) return rc;
    if (!gz || !xhat || !ghat || !dghat || (need_dx && !dx)) return NC_ERR_INVALID_ARGUMENT;
    if (ws_bytes < nc_fftconv_bwd_workspace_size(B, M, fft_h, fft_w) || !ws)
        return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
#define NC_CALL(A, Bv)                                                                     \
    launch_bwd<A, Bv>(st, B, M, hin, win, hout, wout, pad_h, pad_w, gz, xhat, ghat, need_dx, \
                      dx, dghat, accumulate, conj_dghat, ws)
    NC_DISPATCH_FFT(fft_h, fft_w, NC_CALL);
#undef NC_CALL
}

}  // extern "C"

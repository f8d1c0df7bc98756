// Direct (spatial) Green's-function correlation for small filters (Kh * Kw <= 64): the
// reference's conv2d_batched_nchw / small-kernel path (kernels_greens.py:84-123, 177-217;
// propagator.py:373-386, 521-540), where a 3 x 3 filter on a 64 x 64 spectral grid would do
// almost all of its transform work on padding.
//
// Correlation convention (the same as the spectral entry points with window offset p):
//   z[b, m, i, j] = sum over u < kh, v < kw of x[b, i + oh + u, j + ow + v] * G[m, u, v]
// with (oh, ow) = p - (k - 1): (-(kh-1)/2, -(kw-1)/2) for a SAME ROI step, (r0, c0) for the
// VALID full-grid step, (0, 0) for the hoisted border conv.  x is zero outside its plane, or
// read modulo the plane (circular, the CIRCULAR padding mode).  The input may be given as
// n_parts partial planes whose sum is x (the epilogue's direction-group partials).
//
// Each workgroup owns a band of TR output rows of one sample and stages the band's input
// rows (with the filter halo) and the filters in LDS; the reverse stages the cotangent band of
// every direction.  The filter gradient is a fixed-order two-stage reduction: each workgroup
// writes its partial (M, kh, kw) row, nc_rows_sum adds the rows.  No atomics.
#include "nc_common.h"

namespace {

constexpr int kDNT = 256;
constexpr int kDMaxK = 64;      // kh * kw
constexpr int kDMaxM = 64;
constexpr int kDMaxW = 256;     // plane width
constexpr size_t kDLds = 64 * 1024;

NC_DEV int wrapi(int i, int n) {
    i %= n;
    return i < 0 ? i + n : i;
}

// Loads x[b, r, c] (summed over the n_parts partial planes), zero or wrapped outside.
NC_DEV float ld_x(const float* __restrict__ x, int n_parts, size_t pstride, int b, int r, int c,
                  int hin, int win, int circ) {
    if (circ) {
        r = wrapi(r, hin);
        c = wrapi(c, win);
    } else if (r < 0 || r >= hin || c < 0 || c >= win) {
        return 0.f;
    }
    const float* p = x + ((size_t)b * hin + r) * win + c;
    float v = p[0];
    for (int q = 1; q < n_parts; ++q) v += p[q * pstride];
    return v;
}

// Forward: grid (bands, B).  LDS: filters (M*K), then the input band (TR + kh - 1) rows of
// (wout + kw - 1) columns.
__global__ __launch_bounds__(kDNT) void k_dconv_fwd(int M, int hin, int win, int hout, int wout,
                                                    int oh, int ow, int kh, int kw, int circ,
                                                    int TR, const float* __restrict__ x,
                                                    int n_parts, size_t pstride,
                                                    const float* __restrict__ g,
                                                    float* __restrict__ z) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int K = kh * kw;
    float* gs = lds;
    float* xs = lds + M * K;
    const int b = blockIdx.y, i0 = blockIdx.x * TR, tid = threadIdx.x;
    const int rows = min(TR, hout - i0);
    const int xr = rows + kh - 1, xc = wout + kw - 1;
    for (int e = tid; e < M * K; e += kDNT) gs[e] = g[e];
    for (int e = tid; e < xr * xc; e += kDNT) {
        const int r = e / xc, c = e - r * xc;
        xs[e] = ld_x(x, n_parts, pstride, b, i0 + oh + r, ow + c, hin, win, circ);
    }
    __syncthreads();
    for (int e = tid; e < rows * wout; e += kDNT) {
        const int i = e / wout, j = e - i * wout;
        const float* xw = xs + i * xc + j;
        for (int m = 0; m < M; ++m) {
            const float* gm = gs + m * K;
            float acc = 0.f;
            for (int u = 0; u < kh; ++u)
                for (int v = 0; v < kw; ++v) acc = fmaf(xw[u * xc + v], gm[u * kw + v], acc);
            z[(((size_t)b * M + m) * hout + i0 + i) * wout + j] = acc;
        }
    }
}

// Reverse, input gradient: grid (bands of the input rows, B).
//   dx[b, y, c] = sum over m, u, v of gz[b, m, y - oh - u, c - ow - v] * G[m, u, v]
// LDS: filters, then each direction's cotangent band (TR + kh - 1) x (win + kw - 1).
__global__ __launch_bounds__(kDNT) void k_dconv_dx(int M, int hin, int win, int hout, int wout,
                                                   int oh, int ow, int kh, int kw, int circ,
                                                   int TR, const float* __restrict__ gz,
                                                   const float* __restrict__ g,
                                                   float* __restrict__ dx) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int K = kh * kw;
    float* gs = lds;
    float* zs = lds + M * K;
    const int b = blockIdx.y, y0 = blockIdx.x * TR, tid = threadIdx.x;
    const int rows = min(TR, hin - y0);
    const int zr = rows + kh - 1, zc = win + kw - 1;
    const int r_lo = y0 - oh - (kh - 1), c_lo = -ow - (kw - 1);
    for (int e = tid; e < M * K; e += kDNT) gs[e] = g[e];
    for (int e = tid; e < M * zr * zc; e += kDNT) {
        const int m = e / (zr * zc), rc = e - m * zr * zc, r = rc / zc, c = rc - r * zc;
        int ii = r_lo + r, jj = c_lo + c;
        float v = 0.f;
        if (circ) {
            ii = wrapi(ii, hout);
            jj = wrapi(jj, wout);
            v = gz[(((size_t)b * M + m) * hout + ii) * wout + jj];
        } else if (ii >= 0 && ii < hout && jj >= 0 && jj < wout) {
            v = gz[(((size_t)b * M + m) * hout + ii) * wout + jj];
        }
        zs[e] = v;
    }
    __syncthreads();
    for (int e = tid; e < rows * win; e += kDNT) {
        const int y = e / win, c = e - y * win;
        float acc = 0.f;
        for (int m = 0; m < M; ++m) {
            const float* gm = gs + m * K;
            const float* zm = zs + m * zr * zc;
            for (int u = 0; u < kh; ++u)
                for (int v = 0; v < kw; ++v)
                    acc = fmaf(zm[(y + kh - 1 - u) * zc + (c + kw - 1 - v)], gm[u * kw + v], acc);
        }
        dx[((size_t)b * hin + y0 + y) * win + c] = acc;
    }
}

// Reverse, filter gradient partials: grid (bands of the output rows, B); workgroup (band, b)
// writes row (b * bands + band) of part (rows, M*K):
//   part[m, u, v] = sum over the band's pixels (i, j) of gz[b, m, i, j] * x[b, i+oh+u, j+ow+v]
// (pixels in increasing order).  Thread e < M*K owns one filter tap.
__global__ __launch_bounds__(kDNT) void k_dconv_dg(int M, int hin, int win, int hout, int wout,
                                                   int oh, int ow, int kh, int kw, int circ,
                                                   int TR, const float* __restrict__ gz,
                                                   const float* __restrict__ x, int n_parts,
                                                   size_t pstride, float* __restrict__ part) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int K = kh * kw;
    const int b = blockIdx.y, i0 = blockIdx.x * TR, tid = threadIdx.x;
    const int rows = min(TR, hout - i0);
    const int xr = rows + kh - 1, xc = wout + kw - 1;
    float* xs = lds;
    float* zs = lds + xr * xc;
    for (int e = tid; e < xr * xc; e += kDNT) {
        const int r = e / xc, c = e - r * xc;
        xs[e] = ld_x(x, n_parts, pstride, b, i0 + oh + r, ow + c, hin, win, circ);
    }
    for (int e = tid; e < M * rows * wout; e += kDNT) {
        const int m = e / (rows * wout), p = e - m * rows * wout;
        zs[e] = gz[(((size_t)b * M + m) * hout + i0) * wout + p];
    }
    __syncthreads();
    float* dst = part + ((size_t)b * gridDim.x + blockIdx.x) * M * K;
    for (int e = tid; e < M * K; e += kDNT) {
        const int m = e / K, uv = e - m * K, u = uv / kw, v = uv - u * kw;
        const float* zm = zs + m * rows * wout;
        float acc = 0.f;
        for (int i = 0; i < rows; ++i)
            for (int j = 0; j < wout; ++j)
                acc = fmaf(zm[i * wout + j], xs[(i + u) * xc + j + v], acc);
        dst[e] = acc;
    }
}

// Rows per band that keep a workgroup's LDS within kDLds.
int band_rows(size_t fixed_floats, size_t per_row_floats, size_t halo_rows, int total) {
    int tr = 1;
    while (tr < total && (fixed_floats + (tr * 2 + halo_rows) * per_row_floats) * 4 <= kDLds)
        tr *= 2;
    while (tr > 1 && (fixed_floats + (tr + halo_rows) * per_row_floats) * 4 > kDLds) tr /= 2;
    return tr;
}

bool dconv_ok(int B, int M, int hin, int win, int hout, int wout, int kh, int kw, int circ) {
    return B > 0 && M > 0 && M <= kDMaxM && hin > 0 && win > 0 && hout > 0 && wout > 0 &&
           kh > 0 && kw > 0 && kh * kw <= kDMaxK && win <= kDMaxW && wout <= kDMaxW &&
           (!circ || (hin == hout && win == wout));
}

// LDS floats of each kernel's workgroup at TR rows per band.
size_t fwd_floats(int M, int wout, int kh, int kw, int TR) {
    return (size_t)M * kh * kw + (size_t)(TR + kh - 1) * (wout + kw - 1);
}
size_t dx_floats(int M, int win, int kh, int kw, int TR) {
    return (size_t)M * kh * kw + (size_t)M * (TR + kh - 1) * (win + kw - 1);
}
size_t dg_floats(int M, int wout, int kh, int kw, int TR) {
    return (size_t)(TR + kh - 1) * (wout + kw - 1) + (size_t)M * TR * wout;
}

}  // namespace

extern "C" {

int nc_direct_conv_fits(int M, int hin, int win, int hout, int wout, int kh, int kw,
                        int circular, int reverse) {
    if (!dconv_ok(1, M, hin, win, hout, wout, kh, kw, circular)) return 0;
    if (fwd_floats(M, wout, kh, kw, 1) * 4 > kDLds) return 0;
    if (reverse && (dx_floats(M, win, kh, kw, 1) * 4 > kDLds ||
                    dg_floats(M, wout, kh, kw, 1) * 4 > kDLds))
        return 0;
    return 1;
}

int nc_direct_conv_fwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int oh,
                       int ow, int kh, int kw, int circular, const float* x, int n_parts,
                       const float* filters, float* z) {
    if (!dconv_ok(B, M, hin, win, hout, wout, kh, kw, circular) || !x || n_parts <= 0 ||
        !filters || !z)
        return NC_ERR_INVALID_ARGUMENT;
    const int TR = band_rows((size_t)M * kh * kw, wout + kw - 1, kh - 1, hout);
    const size_t shm = fwd_floats(M, wout, kh, kw, TR) * sizeof(float);
    if (shm > kDLds) return NC_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(k_dconv_fwd, dim3((hout + TR - 1) / TR, B), dim3(kDNT), shm,
                       nc_stream(stream), M, hin, win, hout, wout, oh, ow, kh, kw, circular, TR,
                       x, n_parts, (size_t)B * hin * win, filters, z);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_direct_conv_dg_partials(int B, int M, int hout, int wout, int kh, int kw) {
    if (B <= 0 || M <= 0 || hout <= 0 || wout <= 0 || kh <= 0 || kw <= 0) return 0;
    const int xc = wout + kw - 1;
    const int TR = band_rows(0, xc + (size_t)M * wout, kh - 1, hout);
    return B * ((hout + TR - 1) / TR);
}

int nc_direct_conv_bwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int oh,
                       int ow, int kh, int kw, int circular, const float* gz, const float* x,
                       int n_parts, const float* filters, int need_dx, float* dx,
                       float* dg_parts) {
    if (!dconv_ok(B, M, hin, win, hout, wout, kh, kw, circular) || !gz || !x || n_parts <= 0 ||
        !filters || (need_dx && !dx) || !dg_parts)
        return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    const int K = kh * kw;
    if (need_dx) {
        const int zc = win + kw - 1;
        const int TR = band_rows((size_t)M * K, (size_t)M * zc, kh - 1, hin);
        const size_t shm = dx_floats(M, win, kh, kw, TR) * sizeof(float);
        if (shm > kDLds) return NC_ERR_UNSUPPORTED;
        hipLaunchKernelGGL(k_dconv_dx, dim3((hin + TR - 1) / TR, B), dim3(kDNT), shm, st, M, hin,
                           win, hout, wout, oh, ow, kh, kw, circular, TR, gz, filters, dx);
        NC_CHECK_LAUNCH();
    }
    const int TR = band_rows(0, wout + kw - 1 + (size_t)M * wout, kh - 1, hout);
    const size_t shm = dg_floats(M, wout, kh, kw, TR) * sizeof(float);
    if (shm > kDLds) return NC_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(k_dconv_dg, dim3((hout + TR - 1) / TR, B), dim3(kDNT), shm, st, M, hin, win,
                       hout, wout, oh, ow, kh, kw, circular, TR, gz, x, n_parts,
                       (size_t)B * hin * win, dg_parts);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

}  // extern "C"

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
// Tiling.  The forward and the input gradient lay a workgroup's 256 threads over an output
// band as (row group, column): thread (g, j) owns R consecutive rows of column j, so a band is
// TR = R * (256 / width) rows.  The forward stages the band's input rows (with the filter halo)
// and a chunk of MC directions' filters (tap-major) in LDS and keeps MC x R accumulators in
// registers: per tap, R input loads and one broadcast filter vector feed MC * R FMAs.  The
// input gradient stages the cotangent band of a chunk of directions at a time.  The filter
// gradient is an (M x pixels) by (pixels x taps) product per band: each thread owns a 4
// direction x 8 tap register tile over one slice of the band's pixels, the slices are summed
// in LDS in a fixed order and each workgroup writes one (M, kh, kw) partial row; nc_rows_sum
// adds the rows.  No atomics.
#include "nc_common.h"

namespace {

constexpr int kDNT = 256;
constexpr int kDMaxK = 64;      // kh * kw
constexpr int kDMaxM = 64;
constexpr int kDMaxW = 256;     // plane width
constexpr size_t kDLds = 64 * 1024;
constexpr int kGT = 4;          // filter-gradient tile: directions
constexpr int kKT = 8;          //                        taps

NC_DEV int wrapi(int i, int n) {
    while (i < 0) i += n;
    while (i >= n) i -= n;
    return i;
}

// Stages an np x nr x w block (planes, rows, columns): element e = tid, tid + kDNT, ... is
// (m, r, c) = load(m, r, c), stored by store(m, r, c, v).  The thread's first (m, r, c) takes
// one division, the kDNT steps are carried without dividing, and U loads are issued before
// their stores, so each thread keeps U global loads in flight.
template <int U, typename L, typename S>
NC_DEV void stage3(int np, int nr, int w, int tid, L&& load, S&& store) {
    const int dr = kDNT / w, dc = kDNT - dr * w;
    int m = 0, r = tid / w, c = tid - r * w;
    while (r >= nr) {
        r -= nr;
        ++m;
    }
    while (m < np) {
        float v[U];
        int mm[U], rr[U], cc[U];
#pragma unroll
        for (int q = 0; q < U; ++q) {
            mm[q] = m;
            rr[q] = r;
            cc[q] = c;
            v[q] = m < np ? load(m, r, c) : 0.f;
            r += dr;
            c += dc;
            if (c >= w) {
                c -= w;
                ++r;
            }
            while (r >= nr) {
                r -= nr;
                ++m;
            }
        }
#pragma unroll
        for (int q = 0; q < U; ++q)
            if (mm[q] < np) store(mm[q], rr[q], cc[q], v[q]);
    }
}

// x[b, r, c] of a plane given as n_parts partial planes pstride floats apart (summed), zero
// outside the plane or wrapped round it (circular).
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

// Filter rows are padded to kwp = kw rounded up to 4 taps (zero weights), so the tap loops
// run four taps at a time: each step issues all its LDS loads before its FMAs.  The staged
// bands are widened to match (the extra columns hold finite plane values or zeros, which meet
// the zero weights).
NC_DEV int pad4(int v) { return (v + 3) & ~3; }

// Forward: grid (bands, direction chunks, B).  LDS: the chunk's filters, tap-major,
// gT[(u * kwp + v) * MC + m], then the input band: TR + kh - 1 rows of wout + kwp - 1 columns.
template <int R, int MC>
__global__ __launch_bounds__(kDNT) void k_dconv_fwd(int M, int hin, int win, int hout, int wout,
                                                    int oh, int ow, int kh, int kw, int circ,
                                                    int TR, const float* __restrict__ x,
                                                    int n_parts, size_t pstride,
                                                    const float* __restrict__ g,
                                                    float* __restrict__ z) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int K = kh * kw, kwp = pad4(kw), nt = kh * kwp * MC;
    float* gT = lds;
    float* xs = lds + nt;
    const int b = blockIdx.z, m0 = blockIdx.y * MC, i0 = blockIdx.x * TR, tid = threadIdx.x;
    const int rows = min(TR, hout - i0);
    const int xr = rows + kh - 1, xc = wout + kwp - 1;
    for (int e = tid; e < nt; e += kDNT) {
        const int t = e / MC, m = e - t * MC, u = t / kwp, v = t - u * kwp;
        gT[e] = v < kw && m0 + m < M ? g[(size_t)(m0 + m) * K + u * kw + v] : 0.f;
    }
    stage3<4>(
        1, xr, xc, tid,
        [&](int, int r, int c) {
            return ld_x(x, n_parts, pstride, b, i0 + oh + r, ow + c, hin, win, circ);
        },
        [&](int, int r, int c, float v) { xs[r * xc + c] = v; });
    __syncthreads();
    const int j = tid % wout, rb = (tid / wout) * R;
    if (rb >= rows) return;  // idle row groups (no barrier follows)
    float acc[MC][R];
#pragma unroll
    for (int m = 0; m < MC; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
    // rows rb + r + u stay below TR + kh - 1 (the band's allocation); rows past the staged
    // ones only feed outputs r >= rows, which are not stored
    // the (u, four-tap chunk) steps as one loop, unrolled so that a step's loads overlap the
    // previous step's FMAs
    const int nq = kwp >> 2;
    int u = 0, v0 = 0;
#pragma unroll 2
    for (int t = 0; t < kh * nq; ++t) {
        const float* xu = xs + (rb + u) * xc + j + v0;
        const float* gu = gT + (u * kwp + v0) * MC;
        float xv[4][R], gv[4][MC];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int r = 0; r < R; ++r) xv[q][r] = xu[r * xc + q];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int m = 0; m < MC; ++m) gv[q][m] = gu[q * MC + m];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int m = 0; m < MC; ++m)
#pragma unroll
                for (int r = 0; r < R; ++r) acc[m][r] = fmaf(xv[q][r], gv[q][m], acc[m][r]);
        v0 += 4;
        if (v0 == kwp) {
            v0 = 0;
            ++u;
        }
    }
#pragma unroll
    for (int m = 0; m < MC; ++m) {
        if (m0 + m >= M) break;
        float* zm = z + (((size_t)b * M + m0 + m) * hout + i0 + rb) * wout + j;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (rb + r < rows) zm[(size_t)r * wout] = acc[m][r];
    }
}

// Reverse, input gradient: grid (bands of the input rows, B).
//   dx[b, y, c] = sum over m, u, v of gz[b, m, y - oh - u, c - ow - v] * G[m, u, v]
// LDS: the filters gs[(m * kh + u) * kwp + v], then MCH directions' cotangent bands, staged
// chunk by chunk: TR + kh - 1 rows of win + kwp - 1 columns, staged row rz / column cz holding
// gz row y0 - oh - (kh - 1) + rz, column -ow - (kwp - 1) + cz; with NQ > 1 then NQ x PT x R
// floats for the direction groups' partial sums.  The workgroup's PT = 256 / NQ pixel
// threads are laid over the band as (row group, column), R rows each; thread group q < NQ
// takes directions m = q, q + NQ, ... of every chunk, and the NQ partial sums of a pixel
// are added in increasing q.  NQ = 4 on planes up to 64 wide gives four times the
// workgroups of NQ = 1 at the same work per pixel.
template <int R, int NQ>
__global__ __launch_bounds__(kDNT) void k_dconv_dx(int M, int hin, int win, int hout, int wout,
                                                   int oh, int ow, int kh, int kw, int circ,
                                                   int TR, int MCH, const float* __restrict__ gz,
                                                   const float* __restrict__ g,
                                                   float* __restrict__ dx) {
    HIP_DYNAMIC_SHARED(float, lds)
    constexpr int PT = kDNT / NQ;
    const int kwp = pad4(kw), ng = M * kh * kwp;
    const int b = blockIdx.y, y0 = blockIdx.x * TR, tid = threadIdx.x;
    const int rows = min(TR, hin - y0);
    const int zr = rows + kh - 1, zc = win + kwp - 1, zplane = (TR + kh - 1) * zc;
    float* gs = lds;
    float* zs = lds + ng;
    float* red = zs + (size_t)MCH * zplane;
    const int r_lo = y0 - oh - (kh - 1), c_lo = -ow - (kwp - 1);
    for (int e = tid; e < ng; e += kDNT) {
        const int t = e / kwp, v = e - t * kwp;  // t = m * kh + u
        gs[e] = v < kw ? g[(size_t)t * kw + v] : 0.f;
    }
    const int pt = tid % PT, q = tid / PT;
    const int j = pt % win, rb = (pt / win) * R;
    const bool active = rb < rows;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    for (int mc = 0; mc < M; mc += MCH) {
        const int nm = min(MCH, M - mc);
        __syncthreads();  // the previous chunk's reads are done
        const float* gzc = gz + ((size_t)b * M + mc) * hout * wout;
        stage3<8>(
            nm, zr, zc, tid,
            [&](int m, int r, int c) {
                int ii = r_lo + r, jj = c_lo + c;
                if (circ) {
                    ii = wrapi(ii, hout);
                    jj = wrapi(jj, wout);
                } else if (ii < 0 || ii >= hout || jj < 0 || jj >= wout) {
                    return 0.f;
                }
                return gzc[((size_t)m * hout + ii) * wout + jj];
            },
            [&](int m, int r, int c, float v) { zs[m * zplane + r * zc + c] = v; });
        __syncthreads();
        if (!active) continue;
        // taps outside, directions inside (unrolled: the directions' loads are independent)
        const float* z0 = zs + (rb + kh - 1) * zc + j + kwp - 1;
        const float* g0 = gs + (size_t)mc * kh * kwp;
        for (int u = 0; u < kh; ++u) {
            for (int v0 = 0; v0 < kwp; v0 += 4) {
                const float* zu = z0 - u * zc - v0;
                const float* gu = g0 + u * kwp + v0;
#pragma unroll 4
                for (int m = q; m < nm; m += NQ) {
                    float zv[4][R], gv[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) gv[e] = gu[m * kh * kwp + e];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int r = 0; r < R; ++r) zv[e][r] = zu[m * zplane + r * zc - e];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int r = 0; r < R; ++r) acc[r] = fmaf(zv[e][r], gv[e], acc[r]);
                }
            }
        }
    }
    if constexpr (NQ > 1) {
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r) red[(q * PT + pt) * R + r] = acc[r];
        __syncthreads();
        if (q != 0) return;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = red[pt * R + r];
#pragma unroll
            for (int q2 = 1; q2 < NQ; ++q2) v += red[(q2 * PT + pt) * R + r];
            acc[r] = v;
        }
    }
    if (!active) return;
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (rb + r < rows) dx[((size_t)b * hin + y0 + rb + r) * win + j] = acc[r];
}

// Reverse, filter-gradient partials: grid (bands of the output rows, B); workgroup (band, b)
// writes row (b * bands + band) of part (rows, M*K):
//   part[m, u, v] = sum over the band's pixels (i, j) of gz[b, m, i, j] * x[b, i+oh+u, j+ow+v]
// Thread tile (kGT directions x kKT taps) over pixel slice s (pixels s, s + S, ...); the S
// slices are added in increasing s.  LDS: the input band (TR + kh - 1) x (wout + kw - 1) and
// the cotangent band M x TR x wout, then the slices' tiles.
__global__ __launch_bounds__(kDNT) void k_dconv_dg(int M, int hin, int win, int hout, int wout,
                                                   int oh, int ow, int kh, int kw, int circ,
                                                   int TR, const float* __restrict__ gz,
                                                   const float* __restrict__ x, int n_parts,
                                                   size_t pstride, float* __restrict__ part) {
    HIP_DYNAMIC_SHARED(float, lds)
    const int K = kh * kw;
    const int b = blockIdx.y, i0 = blockIdx.x * TR, tid = threadIdx.x;
    const int rows = min(TR, hout - i0);
    const int xr = rows + kh - 1, xc = wout + kw - 1, np = rows * wout;
    float* xs = lds;
    float* zs = lds + xr * xc;
    stage3<4>(
        1, xr, xc, tid,
        [&](int, int r, int c) {
            return ld_x(x, n_parts, pstride, b, i0 + oh + r, ow + c, hin, win, circ);
        },
        [&](int, int r, int c, float v) { xs[r * xc + c] = v; });
    const float* gzb = gz + ((size_t)b * M * hout + i0) * wout;
    stage3<8>(
        M, rows, wout, tid,
        [&](int m, int r, int c) { return gzb[((size_t)m * hout + r) * wout + c]; },
        [&](int m, int r, int c, float v) { zs[(m * rows + r) * wout + c] = v; });
    __syncthreads();
    const int nkt = (K + kKT - 1) / kKT, nroles = ((M + kGT - 1) / kGT) * nkt;
    const int S = kDNT / nroles, role = tid % nroles, s = tid / nroles;
    const int mb = (role / nkt) * kGT, kb = (role % nkt) * kKT;
    int xo[kKT], zo[kGT];
#pragma unroll
    for (int q = 0; q < kKT; ++q) {
        const int k = min(kb + q, K - 1), u = k / kw;
        xo[q] = u * xc + (k - u * kw);
    }
#pragma unroll
    for (int q = 0; q < kGT; ++q) zo[q] = min(mb + q, M - 1) * np;
    float acc[kGT][kKT];
#pragma unroll
    for (int a = 0; a < kGT; ++a)
#pragma unroll
        for (int q = 0; q < kKT; ++q) acc[a][q] = 0.f;
    if (s < S) {
        const int di = S / wout, dj = S - di * wout;
        int i = s / wout, jj = s - i * wout;
#pragma unroll 2
        for (int p = s; p < np; p += S) {
            const int base = i * xc + jj;
            float xv[kKT], zv[kGT];
#pragma unroll
            for (int q = 0; q < kKT; ++q) xv[q] = xs[base + xo[q]];
#pragma unroll
            for (int a = 0; a < kGT; ++a) zv[a] = zs[zo[a] + p];
#pragma unroll
            for (int a = 0; a < kGT; ++a)
#pragma unroll
                for (int q = 0; q < kKT; ++q) acc[a][q] = fmaf(zv[a], xv[q], acc[a][q]);
            i += di;
            jj += dj;
            if (jj >= wout) {
                jj -= wout;
                ++i;
            }
        }
    }
    __syncthreads();  // the staged bands are dead: the slices' tiles reuse the LDS
    constexpr int kTile = kGT * kKT;
    float* red = lds;
    if (s < S) {
#pragma unroll
        for (int a = 0; a < kGT; ++a)
#pragma unroll
            for (int q = 0; q < kKT; ++q) red[(s * nroles + role) * kTile + a * kKT + q] = acc[a][q];
    }
    __syncthreads();
    float* dst = part + ((size_t)b * gridDim.x + blockIdx.x) * M * K;
    for (int e = tid; e < M * K; e += kDNT) {
        const int m = e / K, k = e - m * K;
        const int rl = (m / kGT) * nkt + k / kKT, q = (m % kGT) * kKT + k % kKT;
        float v = 0.f;
        for (int t = 0; t < S; ++t) v += red[(t * nroles + rl) * kTile + q];
        dst[e] = v;
    }
}

bool dconv_ok(int B, int M, int hin, int win, int hout, int wout, int kh, int kw, int circ) {
    return B > 0 && B <= 65535 && M > 0 && M <= kDMaxM && hin > 0 && win > 0 && hout > 0 && wout > 0 &&
           kh > 0 && kw > 0 && kh * kw <= kDMaxK && win <= kDMaxW && wout <= kDMaxW &&
           (!circ || (hin == hout && win == wout));
}

// Launch shapes.  Forward: the register tile (R rows x MC directions) is the first of
// (4, MC), (2, MC), (2, 4) [MC = 8 only] whose grid reaches 2048 workgroups, else the last that
// fits the LDS; MC = 1, 4 or 8 by M.
struct FwdShape {
    int R, MC, TR, bands, chunks;
    size_t shm;
};

int pad4h(int v) { return (v + 3) & ~3; }

size_t fwd_bytes(int MC, int kh, int kw, int TR, int wout) {
    const int kwp = pad4h(kw);
    return ((size_t)kh * kwp * MC + (size_t)(TR + kh - 1) * (wout + kwp - 1)) * 4;
}

bool fwd_shape(int B, int M, int hout, int wout, int kh, int kw, FwdShape* f) {
    const int ngrp = kDNT / wout;
    const int mcs = M == 1 ? 1 : M <= 4 ? 4 : 8;
    const int cand[3][2] = {{4, mcs}, {2, mcs}, {2, 4}};
    bool found = false;
    for (int q = 0; q < (mcs == 8 ? 3 : 2); ++q) {
        const int R = cand[q][0], MC = cand[q][1], TR = ngrp * R;
        const size_t shm = fwd_bytes(MC, kh, kw, TR, wout);
        if (shm > kDLds) continue;
        *f = FwdShape{R, MC, TR, (hout + TR - 1) / TR, (M + MC - 1) / MC, shm};
        found = true;
        if ((size_t)B * f->bands * f->chunks >= 2048) break;
    }
    return found;
}

// Input gradient: NQ = 4 direction groups on planes up to 64 wide (else 1); R = 4, 2 or 1,
// the first whose grid reaches 1024 workgroups (else the last that fits); MCH directions per
// staged chunk, as many as the LDS holds.
struct DxShape {
    int R, NQ, TR, bands, MCH;
    size_t shm;
};

bool dx_shape(int B, int M, int hin, int win, int kh, int kw, DxShape* d) {
    const size_t ng = (size_t)M * kh * pad4h(kw);
    const int NQ = win <= 64 ? 4 : 1, ngrp = (kDNT / NQ) / win;
    const int zc = win + pad4h(kw) - 1;
    bool found = false;
    for (int R = 4; R >= 1; R /= 2) {
        const int TR = ngrp * R;
        const size_t plane = (size_t)(TR + kh - 1) * zc;
        const size_t red = NQ > 1 ? (size_t)kDNT * R : 0;
        if ((ng + red) * 4 >= kDLds) return found;
        const size_t room = kDLds / 4 - ng - red;
        if (room < plane) continue;
        const int MCH = (int)std::min<size_t>(M, room / plane);
        *d = DxShape{R, NQ, TR, (hin + TR - 1) / TR, MCH, (ng + MCH * plane + red) * 4};
        found = true;
        if ((size_t)B * d->bands >= 1024) break;
    }
    return found;
}

// Filter gradient: the band rows that fit the LDS, halved while the grid is under 1024
// workgroups (down to 4 rows).
size_t dg_bytes(int M, int wout, int kh, int kw, int TR) {
    const size_t stage = ((size_t)(TR + kh - 1) * (wout + kw - 1) + (size_t)M * TR * wout) * 4;
    return std::max<size_t>(stage, (size_t)kDNT * kGT * kKT * 4);
}

int dg_rows(int B, int M, int hout, int wout, int kh, int kw) {
    int tr = hout;
    while (tr > 1 && dg_bytes(M, wout, kh, kw, tr) > kDLds) tr = (tr + 1) / 2;
    if (dg_bytes(M, wout, kh, kw, tr) > kDLds) return 0;
    while (tr > 4 && (size_t)B * ((hout + tr - 1) / tr) < 512) tr = (tr + 1) / 2;
    return tr;
}

}  // namespace

extern "C" {

int nc_direct_conv_fits(int M, int hin, int win, int hout, int wout, int kh, int kw,
                        int circular, int reverse) {
    if (!dconv_ok(1, M, hin, win, hout, wout, kh, kw, circular)) return 0;
    FwdShape f;
    if (!fwd_shape(1, M, hout, wout, kh, kw, &f)) return 0;
    DxShape d;
    if (reverse && (!dx_shape(1, M, hin, win, kh, kw, &d) || !dg_rows(1, M, hout, wout, kh, kw)))
        return 0;
    return 1;
}

int nc_direct_conv_fwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int oh,
                       int ow, int kh, int kw, int circular, const float* x, int n_parts,
                       const float* filters, float* z) {
    if (!dconv_ok(B, M, hin, win, hout, wout, kh, kw, circular) || !x || n_parts <= 0 ||
        !filters || !z)
        return NC_ERR_INVALID_ARGUMENT;
    FwdShape f;
    if (!fwd_shape(B, M, hout, wout, kh, kw, &f)) return NC_ERR_UNSUPPORTED;
    const dim3 grid(f.bands, f.chunks, B);
    const size_t ps = (size_t)B * hin * win;
#define NC_DFWD(R_, MC_)                                                                       \
    hipLaunchKernelGGL((k_dconv_fwd<R_, MC_>), grid, dim3(kDNT), f.shm, nc_stream(stream), M,   \
                       hin, win, hout, wout, oh, ow, kh, kw, circular, f.TR, x, n_parts, ps,   \
                       filters, z)
    if (f.R == 4) {
        if (f.MC == 8) NC_DFWD(4, 8);
        else if (f.MC == 4) NC_DFWD(4, 4);
        else NC_DFWD(4, 1);
    } else {
        if (f.MC == 8) NC_DFWD(2, 8);
        else if (f.MC == 4) NC_DFWD(2, 4);
        else NC_DFWD(2, 1);
    }
#undef NC_DFWD
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_direct_conv_dg_partials(int B, int M, int hout, int wout, int kh, int kw) {
    if (B <= 0 || M <= 0 || hout <= 0 || wout <= 0 || kh <= 0 || kw <= 0) return 0;
    const int TR = dg_rows(B, M, hout, wout, kh, kw);
    return TR ? B * ((hout + TR - 1) / TR) : 0;
}

int nc_direct_conv_bwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int oh,
                       int ow, int kh, int kw, int circular, const float* gz, const float* x,
                       int n_parts, const float* filters, int need_dx, float* dx,
                       float* dg_parts) {
    if (!dconv_ok(B, M, hin, win, hout, wout, kh, kw, circular) || !gz || !x || n_parts <= 0 ||
        !filters || (need_dx && !dx) || !dg_parts)
        return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    const int TR = dg_rows(B, M, hout, wout, kh, kw);
    DxShape d;
    if (!TR || (need_dx && !dx_shape(B, M, hin, win, kh, kw, &d))) return NC_ERR_UNSUPPORTED;
    if (need_dx) {
        const dim3 grid(d.bands, B);
#define NC_DDX(R_, NQ_)                                                                        \
    hipLaunchKernelGGL((k_dconv_dx<R_, NQ_>), grid, dim3(kDNT), d.shm, st, M, hin, win, hout,   \
                       wout, oh, ow, kh, kw, circular, d.TR, d.MCH, gz, filters, dx)
        if (d.NQ == 4) {
            if (d.R == 4) NC_DDX(4, 4);
            else if (d.R == 2) NC_DDX(2, 4);
            else NC_DDX(1, 4);
        } else {
            if (d.R == 4) NC_DDX(4, 1);
            else if (d.R == 2) NC_DDX(2, 1);
            else NC_DDX(1, 1);
        }
#undef NC_DDX
        NC_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(k_dconv_dg, dim3((hout + TR - 1) / TR, B), dim3(kDNT),
                       dg_bytes(M, wout, kh, kw, TR), st, M, hin, win, hout, wout, oh, ow, kh,
                       kw, circular, TR, gz, x, n_parts, (size_t)B * hin * win, dg_parts);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

}  // extern "C"

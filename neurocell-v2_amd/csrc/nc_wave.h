// Wavefront-level 2D real FFTs for (FH x FW) spectral grids, FH, FW in {16, 32, 64}.
//
// One 64-lane wavefront owns PPW = 128 / FW planes and needs no block barrier: every 1D
// transform runs entirely inside one lane's registers, and one LDS transposition buffer per
// plane (T, rows x (FW/2 + 1) cpx) moves data between the two passes.
//
//   row pass    lane <-> (plane, row pair): two real rows (q, q + NR) are packed as
//               a + i*b, transformed with one FW-point FFT and split into their half spectra;
//   column pass lane <-> (plane, packed column kc < FW/2): the FH-point FFT of column kc;
//               column 0 carries DC + i*Nyquist (both real-signal spectra, so products with
//               other real-signal spectra keep the packing valid and it unpacks losslessly).
//
// The inverse runs the passes backwards and writes only the requested window of output rows
// and columns, taken circularly from (row0, col0): that gives both the overlap-save crop of
// the forward correlation and the unshifted roll of its adjoint.
#pragma once

#include "nc_fft.h"
#include "nc_wtab.h"

#define NC_DEV_HOST_INLINE __host__ __device__ inline

// v * W_N^e (forward sign; INV conjugates).  e and N are compile-time constants once the
// callers' loops are unrolled, so the branches and the table reads fold away.
template <int N, bool INV>
NC_DEV cpx twm(cpx v, int e) {
    e &= N - 1;
    if (e == 0) return v;
    const int j = e * (64 / N);
    if (j == 16) return INV ? cmul_i(v) : cmul_negi(v);
    if (j == 32) return cmk(-v.x, -v.y);
    if (j == 48) return INV ? cmul_negi(v) : cmul_i(v);
    const float c = kWc64[j], s = INV ? -kWs64[j] : kWs64[j];
    return cmk(v.x * c - v.y * s, v.x * s + v.y * c);
}

template <int N>
struct RegSplit;
template <>
struct RegSplit<16> { static constexpr int N1 = 4, N2 = 4; };
template <>
struct RegSplit<32> { static constexpr int N1 = 8, N2 = 4; };
template <>
struct RegSplit<64> { static constexpr int N1 = 8, N2 = 8; };

// In-register N-point DFT, natural order in and out (n = N2*n1 + n2, k = k1 + N1*k2).
template <int N, bool INV>
NC_DEV void fft_reg(cpx* x) {
    if constexpr (N == 4) {
        dft4<INV>(x[0], x[1], x[2], x[3]);
    } else if constexpr (N == 8) {
        dft8<INV>(x);
    } else {
        constexpr int N1 = RegSplit<N>::N1, N2 = RegSplit<N>::N2;
        cpx y[N];
#pragma unroll
        for (int n2 = 0; n2 < N2; ++n2) {
            cpx t[N1];
#pragma unroll
            for (int n1 = 0; n1 < N1; ++n1) t[n1] = x[N2 * n1 + n2];
            fft_reg<N1, INV>(t);
#pragma unroll
            for (int k1 = 0; k1 < N1; ++k1) y[n2 * N1 + k1] = twm<N, INV>(t[k1], n2 * k1);
        }
#pragma unroll
        for (int k1 = 0; k1 < N1; ++k1) {
            cpx t[N2];
#pragma unroll
            for (int n2 = 0; n2 < N2; ++n2) t[n2] = y[n2 * N1 + k1];
            fft_reg<N2, INV>(t);
#pragma unroll
            for (int k2 = 0; k2 < N2; ++k2) x[k1 + N1 * k2] = t[k2];
        }
    }
}

template <int FH, int FW>
struct WGeo {
    static_assert(FW >= 16 && FW <= 64 && FH >= 16 && FH <= 64, "wave FFT grid");
    static constexpr int SP = FW / 2 + 1;   // half-spectrum row pitch (cpx)
    static constexpr int F = FH * SP;       // half-spectrum size (cpx)
    static constexpr int NC = FW / 2;       // packed columns
    static constexpr int PPW = 64 / NC;     // planes per wavefront
    static constexpr int PITCH = NC + 1;    // LDS pitch of a transposed row (cpx)
    static constexpr int PF = FH * NC;      // packed spectrum size (cpx)
};

// The passes never predicate a store (or a load) per unrolled element: the compiler keeps every
// predicated element's address live and the register count explodes.  Unwanted rows or
// columns go to a trash slot instead, and missing inputs are read from a zero slot.
//
// T layout: plane ps has rows + 2 rows of PITCH cpx: rows [0, rows) of data, row `rows` (the
// trash row) and row `rows + 1` (kept zero by the forward transforms).
template <int FH, int FW>
NC_DEV cpx* trow(cpx* T, int rows, int ps, int r) {
    return T + (ps * (rows + 2) + r) * WGeo<FH, FW>::PITCH;
}

// Input staging: plane p, row r, column c at S[(p * rows + r) * (FW + 1) + c], zero for
// cols <= c < FW (the row pass reads every column of a row, with no per-column select).
NC_DEV_HOST_INLINE int istage_floats(int ppw, int rows, int fw) { return ppw * rows * (fw + 1); }

// Stages np planes of rows x cols floats (plane p at src + p * pstride, contiguous) into S;
// missing planes are zero.  With vec (n = rows*cols and pstride multiples of 4, src 16-byte
// aligned) the loads are float4s; every load of a batch is issued before the LDS scatter, so
// a wavefront keeps many global loads in flight.  FLIP reads each plane rotated by 180
// degrees (the reversed flat order).  NP > 1: each value is the sum of NP partial planes
// qstride floats apart, added in increasing order (NP == 0: nq of them, a runtime count).
template <int FW, int PPW, bool FLIP, int NP = 1>
NC_DEV void istage(const float* __restrict__ src, size_t pstride, int np, int rows, int cols,
                   bool vec, float* S, size_t qstride = 0, int nq = 1) {
    const int nparts = NP == 0 ? nq : NP;
    auto ld = [&](const float* a) {
        float v = a[0];
        if constexpr (NP != 1) {
#pragma unroll
            for (int q = 1; q < (NP == 0 ? 1 : NP); ++q) v += a[q * qstride];
            if constexpr (NP == 0)
                for (int q = 1; q < nparts; ++q) v += a[q * qstride];
        }
        return v;
    };
    auto ld4 = [&](const float4* a) {
        float4 v = a[0];
        if constexpr (NP != 1) {
            auto add = [&](int q) {
                const float4 w = a[q * (qstride >> 2)];
                v.x += w.x;
                v.y += w.y;
                v.z += w.z;
                v.w += w.w;
            };
#pragma unroll
            for (int q = 1; q < (NP == 0 ? 1 : NP); ++q) add(q);
            if constexpr (NP == 0)
                for (int q = 1; q < nparts; ++q) add(q);
        }
        return v;
    };
    const int lane = threadIdx.x & 63;
    const int n = rows * cols;
    // zero padding columns [cols, FW) of every staged row
    const int pad = FW - cols;
    if (pad > 0)
        for (int e = lane; e < PPW * rows * pad; e += 64) {
            const int row = e / pad, c = cols + (e - row * pad);
            S[row * (FW + 1) + c] = 0.f;
        }
    if (!FLIP && vec) {
        constexpr int U = 4;
        const int n4 = n >> 2;
        for (int e0 = lane; e0 < n4; e0 += 64 * U) {
            float4 t[PPW][U];
#pragma unroll
            for (int p = 0; p < PPW; ++p) {
                const float4* s4 = reinterpret_cast<const float4*>(src + p * pstride);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int e = e0 + 64 * u;
                    t[p][u] = (p < np && e < n4) ? ld4(s4 + e) : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = e0 + 64 * u;
                if (e < n4) {
                    const int r0 = (4 * e) / cols;
                    const int c0 = 4 * e - r0 * cols;
#pragma unroll
                    for (int p = 0; p < PPW; ++p) {
                        const float vals[4] = {t[p][u].x, t[p][u].y, t[p][u].z, t[p][u].w};
                        int r = r0, c = c0;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            S[(p * rows + r) * (FW + 1) + c] = vals[k];
                            if (++c == cols) {
                                c = 0;
                                ++r;
                            }
                        }
                    }
                }
            }
        }
        return;
    }
    constexpr int U = 8;
    for (int e0 = lane; e0 < n; e0 += 64 * U) {
        float t[PPW][U];
#pragma unroll
        for (int p = 0; p < PPW; ++p)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = e0 + 64 * u;
                t[p][u] = (p < np && e < n) ? ld(src + p * pstride + (FLIP ? n - 1 - e : e)) : 0.f;
            }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = e0 + 64 * u;
            if (e < n) {
                const int r = e / cols, c = e - r * cols;
#pragma unroll
                for (int p = 0; p < PPW; ++p) S[(p * rows + r) * (FW + 1) + c] = t[p][u];
            }
        }
    }
}

// Row pass of the forward transform over the staged planes S: writes the packed half-spectrum
// rows to T and zeroes each plane's zero row.  Every lane of the wavefront must call it: a
// barrier separates each pass's loads from its stores, so S may share LDS with T when one
// pass covers all row pairs.
template <int FH, int FW>
NC_DEV void wrow_fwd(const float* S, int rows, cpx* T) {
    using W = WGeo<FH, FW>;
    const int lane = threadIdx.x & 63;
    const int NR = (rows + 1) >> 1;
    const int slots = W::PPW * NR;
    for (int s0 = 0; s0 < slots; s0 += 64) {
        const int s = s0 + lane;
        const bool on = s < slots;
        const int ps = on ? s / NR : 0, q = on ? s - ps * NR : 0, rb = q + NR;
        const bool hb = on && rb < rows;
        const float* sa = S + (ps * rows + q) * (FW + 1);
        const float* sb = S + (ps * rows + (hb ? rb : q)) * (FW + 1);
        const float bs = hb ? 1.f : 0.f;
        cpx v[FW];
#pragma unroll
        for (int c = 0; c < FW; ++c) v[c] = cmk(sa[c], sb[c] * bs);
        __syncthreads();
        if (on) {
            fft_reg<FW, false>(v);
            cpx* ta = trow<FH, FW>(T, rows, ps, q);
            cpx* tb = trow<FH, FW>(T, rows, ps, hb ? rb : rows);
            ta[0] = cmk(v[0].x, v[FW / 2].x);
            tb[0] = cmk(v[0].y, v[FW / 2].y);
#pragma unroll
            for (int k = 1; k < FW / 2; ++k) {
                const cpx A = v[k], Bc = cconj(v[FW - k]);
                ta[k] = cscale(cadd(A, Bc), 0.5f);
                tb[k] = cmul_negi(cscale(csub(A, Bc), 0.5f));
            }
        }
    }
    {
        const int ps = lane / W::NC, kc = lane % W::NC;
        trow<FH, FW>(T, rows, ps, rows + 1)[kc] = cmk(0.f, 0.f);
    }
}

// Column pass of the forward transform: lane (ps, kc) reads column kc of plane ps from T
// (rows [0, rows), the zero row above) and leaves its FH-point spectrum in v.
template <int FH, int FW>
NC_DEV void wcol_fwd(cpx* T, int rows, cpx* v) {
    using W = WGeo<FH, FW>;
    const int lane = threadIdx.x & 63, ps = lane / W::NC, kc = lane % W::NC;
    const cpx* t = trow<FH, FW>(T, rows, ps, 0) + kc;
    int rl = rows;  // a vector copy, so the row selects below stay vector operations
    NC_PIN(rl);
#pragma unroll
    for (int r = 0; r < FH; ++r) v[r] = t[(r < rl ? r : rl + 1) * W::PITCH];
    fft_reg<FH, false>(v);
}

// Column pass of the inverse transform: v holds lane (ps, kc)'s packed spectrum column; output
// rows i = (r - row0) mod FH < rows land in T (the others in the trash row).
template <int FH, int FW>
NC_DEV void wcol_inv(cpx* v, int row0, int rows, cpx* T) {
    using W = WGeo<FH, FW>;
    const int lane = threadIdx.x & 63, ps = lane / W::NC, kc = lane % W::NC;
    fft_reg<FH, true>(v);
    cpx* t = trow<FH, FW>(T, rows, ps, 0) + kc;
#pragma unroll
    for (int r = 0; r < FH; ++r) {
        int i = (r - row0) & (FH - 1);
        i = i < rows ? i : rows;
        t[i * W::PITCH] = v[r];
    }
}

// Output staging of the inverse row pass: plane p, output row i (i < rows; row `rows` of each
// plane is a trash row), window column j at O[(p * (rows + 1) + i) * (FW + 1) + j].  Every
// one of the FW columns is stored, at j = (c - col0) mod FW, so no store is predicated; the
// copy-out takes the first `cols` of each row.
NC_DEV_HOST_INLINE int ostage_floats(int ppw, int rows, int fw) {
    return ppw * (rows + 1) * (fw + 1);
}

// Row pass of the inverse transform: output rows [0, rows) of each plane, times scale, into
// the staging O.  Every lane must call it; a barrier separates each pass's reads of T from its
// stores (which may overwrite T when one pass covers all row pairs).
template <int FH, int FW>
NC_DEV void wrow_inv(cpx* T, int col0, int rows, float scale, float* O) {
    using W = WGeo<FH, FW>;
    const int lane = threadIdx.x & 63;
    const int NR = (rows + 1) >> 1;
    const int slots = W::PPW * NR;
    for (int s0 = 0; s0 < slots; s0 += 64) {
        const int s = s0 + lane;
        const bool on = s < slots;
        const int ps = on ? s / NR : 0, q = on ? s - ps * NR : 0, rb = q + NR;
        const bool hb = on && rb < rows;
        const cpx* ta = trow<FH, FW>(T, rows, ps, q);
        const cpx* tb = trow<FH, FW>(T, rows, ps, hb ? rb : q);
        const float bs = hb ? 1.f : 0.f;
        cpx v[FW];
        {
            const cpx a0 = ta[0], b0 = tb[0];
            v[0] = cmk(a0.x, b0.x * bs);
            v[FW / 2] = cmk(a0.y, b0.y * bs);
#pragma unroll
            for (int k = 1; k < FW / 2; ++k) {
                const cpx A = ta[k], Bv = cscale(tb[k], bs);
                v[k] = cadd(A, cmul_i(Bv));
                v[FW - k] = cadd(cconj(A), cmul_i(cconj(Bv)));
            }
        }
        __syncthreads();
        if (on) {
            fft_reg<FW, true>(v);
            float* oa = O + (ps * (rows + 1) + q) * (FW + 1);
            float* ob = O + (ps * (rows + 1) + (hb ? rb : rows)) * (FW + 1);
            int sh = FW - col0;  // a vector copy, so the column offsets stay vector values
            NC_PIN(sh);
#pragma unroll
            for (int c = 0; c < FW; ++c) {
                const int j = (c + sh) & (FW - 1);
                oa[j] = v[c].x * scale;
                ob[j] = v[c].y * scale;
            }
        }
    }
}

// Copies np staged planes (rows x cols, cols <= FW) to dst, contiguous; each lane moves a column
// of up to 8 rows per batch.
template <int FW>
NC_DEV void ostage_copy(const float* O, int np, int rows, int cols, float* __restrict__ dst) {
    const int lane = threadIdx.x & 63;
    const int rpi = 64 / cols;  // rows per iteration
    const int ri = lane / cols, j = lane - ri * cols;
    if (ri >= rpi) return;
    constexpr int U = 8;
    const int total = np * rows;  // rows over all planes; plane p's row i is staged row g + p
    for (int g0 = ri; g0 < total; g0 += U * rpi) {
        float t[U];
        int gp[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int g = min(g0 + u * rpi, total - 1);
            gp[u] = g;
            t[u] = O[(g + g / rows) * (FW + 1) + j];
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (g0 + u * rpi < total) dst[(size_t)gp[u] * cols + j] = t[u];
    }
}

// Stages the Nyquist column (column FW/2) of the wavefront's PPW half-spectra into NQ[ps][kh]
// with every lane loading FH/NC entries; src(ps) is plane ps's half-spectrum base.  The
// caller barriers before reading NQ.
template <int FH, int FW, class Src>
NC_DEV void stage_nyquist(Src src, cpx* NQ) {
    using W = WGeo<FH, FW>;
    const int lane = threadIdx.x & 63, ps = lane / W::NC, kc = lane % W::NC;
    const cpx* p = src(ps);
    for (int kh = kc; kh < FH; kh += W::NC) NQ[ps * FH + kh] = p[kh * W::SP + FW / 2];
}

// Packed-column products.  For the packed column (kc == 0) v = P + iQ with P, Q the spectra
// (over kh) of the real DC and Nyquist columns; r[kh] is the other operand's column kc (its DC
// column on lane kc == 0) and refN(kh) reads its Nyquist column.  Both operands are
// real-signal spectra there, so the product columns are Hermitian in kh and are re-packed as
// P' + iQ'.  For kc > 0 the product is v[kh] * conj(r[kh]).  The result replaces v.
template <int FH, class RefN>
NC_DEV void packed_mulc(cpx* v, const cpx* r, int kc, RefN refN) {
    if (kc != 0) {
#pragma unroll
        for (int kh = 0; kh < FH; ++kh) v[kh] = cmulc(v[kh], r[kh]);
        return;
    }
#pragma unroll
    for (int kh = 0; kh <= FH / 2; ++kh) {
        const int nk = (FH - kh) & (FH - 1);
        const cpx c = v[kh], d = cconj(v[nk]);
        const cpx P = cscale(cadd(c, d), 0.5f);
        const cpx Q = cmul_negi(cscale(csub(c, d), 0.5f));
        const cpx Pp = cmulc(P, r[kh]), Qp = cmulc(Q, refN(kh));
        v[kh] = cadd(Pp, cmul_i(Qp));
        if (nk != kh) v[nk] = cadd(cconj(Pp), cmul_i(cconj(Qp)));
    }
}

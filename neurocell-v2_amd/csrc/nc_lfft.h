// Workgroup-level 2D real FFTs for spectral grids with an axis of 128 or 256 points
// (FH, FW in {64, 128, 256}), where neither a whole plane nor a 1D transform fits in one
// lane's registers, and a 256 x 129 complex half-spectrum (264 KB) does not fit in LDS.
//
// Each 1D transform is the four-step group FFT of nc_fft.h (G threads holding E values, one
// LDS exchange).  A workgroup of NT threads transforms one plane, keeping only a *segment* of
// the intermediate between the two passes in LDS:
//
//   forward  (real rows -> half-spectrum): the row pass keeps, for every live row pair, the
//            bins of a segment of CS packed columns (and their mirror bins, which the real
//            split needs); the column pass then finishes those CS columns.  A plane whose
//            whole intermediate fits is one segment; otherwise the row transforms are
//            repeated once per segment (grid dimension y).
//   inverse  (half-spectrum -> real window): the column pass runs over every packed column
//            but keeps only a segment of RS output rows; the row pass then finishes those
//            rows.  The column transforms are repeated once per row segment.
//
// Packed column 0 carries DC + i*Nyquist (both spectra of real columns), as in the other
// transforms of this library; inputs past (hin, win) are never read (row pruning) and
// inverse outputs are taken circularly from (row0, col0), which gives both the overlap-save
// crop and the unshifted roll of the adjoint.
#pragma once

#include "nc_fft.h"

template <int FH, int FW, int NT>
struct LGeo {
    static_assert((FH == 64 || FH == 128 || FH == 256) && (FW == 64 || FW == 128 || FW == 256),
                  "large-grid transforms cover 64..256 points per axis");
    static constexpr int SP = FW / 2 + 1;  // half-spectrum row pitch (cpx)
    static constexpr int F = FH * SP;      // half-spectrum size (cpx)
    static constexpr int NC = FW / 2;      // packed columns
    using GH = GroupFft<FH>;
    using GW = GroupFft<FW>;
    static_assert(NT % GH::G == 0 && NT % GW::G == 0, "whole groups");
    static constexpr int NGH = NT / GH::G;  // column transforms in flight
    static constexpr int NGW = NT / GW::G;  // row-pair transforms in flight
    // Column groups interleave lane by lane (group g = tid % NGH, so each 16-lane quarter of
    // a wavefront holds 16 groups at one row t).  The LDS serves 8-byte accesses 16 lanes per
    // pass over 16 bank pairs (a cpx at index a sits in pair a mod 16, as the bank-conflict
    // counters of these passes bear out), so the exchange slots lie SCR_HS cpx apart with
    // SCR_HS odd (1 mod 32): a quarter's 16 groups then hit 16 different pairs, both for the
    // stage-1 writes (row k1, column t) and the stage-2 reads (row t, column t2).
    static constexpr int SCR_HS = GH::SCR + ((1 - GH::SCR % 32) % 32 + 32) % 32;
    static constexpr int SCR_H = NGH * SCR_HS;
    static constexpr int SCR_W = NGW * GW::SCR;
    static constexpr int SCR = SCR_H > SCR_W ? SCR_H : SCR_W;  // exchange scratch (cpx)
};

// LDS (bytes) of the inverse over a segment of `rows` output rows: the segment buffer
// T ((rows + 1) x SP cpx, row `rows` is a trash row), the exchange scratch and the twiddles.
template <int FH, int FW, int NT>
__host__ __device__ constexpr size_t linv_lds_bytes(int rows) {
    using L = LGeo<FH, FW, NT>;
    return ((size_t)NC_TW_N + L::SCR + (size_t)(rows + 1) * L::SP) * sizeof(cpx);
}

// LDS (bytes) of the forward over a segment of cs packed columns for hin live rows: the
// pair buffer Y ((hin + 1)/2 x (2*cs + 1) cpx, the last slot of a pair row is a trash slot),
// the packed-column staging C0 (FH cpx), the exchange scratch and the twiddles.
template <int FH, int FW, int NT>
__host__ __device__ constexpr size_t lfwd_lds_bytes(int hin, int cs) {
    using L = LGeo<FH, FW, NT>;
    return ((size_t)NC_TW_N + L::SCR + FH + (size_t)((hin + 1) / 2) * (2 * cs + 1)) * sizeof(cpx);
}

// Forward transform of one real (hin x win) plane at the origin of the (FH x FW) grid,
// restricted to packed columns [c0, c0 + cs).  load(r, c) is called for r < hin, c < win
// only.  out(kh, kw, value) receives every half-spectrum bin (kh < FH) of the columns
// kw in [c0, c0 + cs), and, for the segment with c0 == 0, also the Nyquist column kw = FW/2.
// All NT threads must call it (it contains barriers and ends with one).
template <int FH, int FW, int NT, class Load, class Out>
NC_DEV void lplane_rfft2(Load load, int hin, int win, int c0, int cs, Out out, cpx* Y, cpx* C0,
                         cpx* scr, const cpx* tw) {
    using L = LGeo<FH, FW, NT>;
    constexpr int EW = L::GW::E, GW = L::GW::G, EH = L::GH::E, GH = L::GH::G;
    const int tid = threadIdx.x;
    const int yp = 2 * cs + 1;  // pair-row pitch; slot 2*cs is the trash slot
    const int npairs = (hin + 1) >> 1;

    // Row pass: lanes of a group take consecutive columns of one row pair.
    for (int p0 = 0; p0 < npairs; p0 += L::NGW) {
        const int g = tid / GW, t = tid % GW, p = p0 + g;
        const bool on = p < npairs;
        cpx* sc = scr + g * L::GW::SCR;
        cpx v[EW];
        if (on) {
            const int ra = 2 * p, rb = 2 * p + 1;
            const bool hasb = rb < hin;
#pragma unroll
            for (int n1 = 0; n1 < EW; ++n1) {
                const int c = t + GW * n1;
                float a = 0.f, b = 0.f;
                if (c < win) {
                    a = load(ra, c);
                    if (hasb) b = load(rb, c);
                }
                v[n1] = cmk(a, b);
            }
            gfft_stage1<FW, false>(v, t, sc, tw);
        }
        __syncthreads();
        if (on) {
            gfft_stage2<FW, false>(v, t, sc);
            cpx* y = Y + p * yp;
#pragma unroll
            for (int s = 0; s < EW; ++s) {
                const int k = L::GW::bin(t, s);
                const int km = (FW - k) & (FW - 1);
                int j = yp - 1;
                if (k >= c0 && k < c0 + cs) j = k - c0;
                else if (k == FW / 2) j = c0 == 0 ? cs : yp - 1;
                else if (k != 0 && km >= c0 && km < c0 + cs) j = cs + (km - c0);
                y[j] = v[s];
            }
        }
        __syncthreads();
    }

    // Column pass: lanes of a wavefront take consecutive columns (coalesced stores).
    for (int j0 = 0; j0 < cs; j0 += L::NGH) {
        const int g = tid % L::NGH, t = tid / L::NGH, jj = j0 + g;
        const bool on = jj < cs;
        const int kw = c0 + jj;
        cpx* sc = scr + g * L::SCR_HS;
        cpx v[EH];
        if (on) {
#pragma unroll
            for (int n1 = 0; n1 < EH; ++n1) {
                const int r = t + GH * n1;
                cpx val = cmk(0.f, 0.f);
                if (r < hin) {
                    const cpx* y = Y + (r >> 1) * yp;
                    const bool odd = r & 1;
                    if (kw == 0) {
                        const cpx z0 = y[0], zn = y[cs];
                        val = odd ? cmk(z0.y, zn.y) : cmk(z0.x, zn.x);
                    } else {
                        const cpx A = y[jj], Bc = cconj(y[cs + jj]);
                        val = odd ? cmul_negi(cscale(csub(A, Bc), 0.5f))
                                  : cscale(cadd(A, Bc), 0.5f);
                    }
                }
                v[n1] = val;
            }
            gfft_stage1<FH, false>(v, t, sc, tw);
        }
        __syncthreads();
        if (on) {
            gfft_stage2<FH, false>(v, t, sc);
#pragma unroll
            for (int s = 0; s < EH; ++s) {
                const int kh = L::GH::bin(t, s);
                if (kw == 0) C0[kh] = v[s];
                else out(kh, kw, v[s]);
            }
        }
        __syncthreads();
    }

    // Unpack the packed column: C = P + iQ with P, Q spectra of the real DC / Nyquist columns.
    if (c0 == 0) {
        for (int kh = tid; kh < FH; kh += NT) {
            const cpx c = C0[kh], cm = cconj(C0[(FH - kh) & (FH - 1)]);
            out(kh, 0, cscale(cadd(c, cm), 0.5f));
            out(kh, FW / 2, cmul_negi(cscale(csub(c, cm), 0.5f)));
        }
        __syncthreads();
    }
}

// Inverse transform (unnormalised inverse times `scale`) of a half-spectrum, materialising
// output rows i = (r - row0) mod FH < rows and columns j = (c - col0) mod FW < cols.
// specp(kh, kw), kw < FW/2, returns packed column values: for kw == 0, DC + i*Nyquist.
// store(i, j, value) receives the outputs.  T: (rows + 1) x SP cpx.  All NT threads must
// call it (it contains barriers and ends with one).
template <int FH, int FW, int NT, class SpecP, class Store>
NC_DEV void lplane_irfft2(SpecP specp, int row0, int rows, int col0, int cols, float scale,
                          Store store, cpx* T, cpx* scr, const cpx* tw) {
    using L = LGeo<FH, FW, NT>;
    constexpr int EW = L::GW::E, GW = L::GW::G, EH = L::GH::E, GH = L::GH::G;
    constexpr int SP = L::SP;
    const int tid = threadIdx.x;

    // Inverse column pass over every packed column; only the segment's rows are kept.
    for (int k0 = 0; k0 < L::NC; k0 += L::NGH) {
        const int g = tid % L::NGH, t = tid / L::NGH, kw = k0 + g;
        const bool on = kw < L::NC;
        cpx* sc = scr + g * L::SCR_HS;
        cpx v[EH];
        if (on) {
#pragma unroll
            for (int n1 = 0; n1 < EH; ++n1) v[n1] = specp(t + GH * n1, kw);
            gfft_stage1<FH, true>(v, t, sc, tw);
        }
        __syncthreads();
        if (on) {
            gfft_stage2<FH, true>(v, t, sc);
#pragma unroll
            for (int s = 0; s < EH; ++s) {
                int i = (L::GH::bin(t, s) - row0) & (FH - 1);
                i = i < rows ? i : rows;
                T[i * SP + kw] = v[s];
            }
        }
        __syncthreads();
    }

    // Inverse row pass on pairs of output rows: z = X_a + i*X_b, one complex transform.
    const int npairs = (rows + 1) >> 1;
    for (int p0 = 0; p0 < npairs; p0 += L::NGW) {
        const int g = tid / GW, t = tid % GW, p = p0 + g;
        const bool on = p < npairs;
        const int ia = 2 * p, ib = 2 * p + 1;
        const bool hasb = ib < rows;
        cpx* sc = scr + g * L::GW::SCR;
        cpx v[EW];
        if (on) {
            const cpx* ta = T + ia * SP;
            const cpx* tb = T + (hasb ? ib : ia) * SP;
            const float bs = hasb ? 1.f : 0.f;
#pragma unroll
            for (int n1 = 0; n1 < EW; ++n1) {
                const int k = t + GW * n1;
                cpx a, b;
                if (n1 < EW / 2) {  // k < FW/2
                    if (k == 0) {
                        a = cmk(ta[0].x, 0.f);
                        b = cmk(tb[0].x, 0.f);
                    } else {
                        a = ta[k];
                        b = tb[k];
                    }
                } else {  // k >= FW/2
                    if (k == FW / 2) {
                        a = cmk(ta[0].y, 0.f);
                        b = cmk(tb[0].y, 0.f);
                    } else {
                        a = cconj(ta[FW - k]);
                        b = cconj(tb[FW - k]);
                    }
                }
                v[n1] = cadd(a, cmul_i(cscale(b, bs)));
            }
            gfft_stage1<FW, true>(v, t, sc, tw);
        }
        __syncthreads();
        if (on) {
            gfft_stage2<FW, true>(v, t, sc);
#pragma unroll
            for (int s = 0; s < EW; ++s) {
                const int j = (L::GW::bin(t, s) - col0) & (FW - 1);
                if (j < cols) {
                    store(ia, j, v[s].x * scale);
                    if (hasb) store(ib, j, v[s].y * scale);
                }
            }
        }
        __syncthreads();
    }
}

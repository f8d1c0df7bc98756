// LDS-resident, row-pruned 2D real FFTs for one plane per workgroup (gfx950, wave64).
//
// A length-N transform (N = E*G, both powers of two) is run by a group of G threads that each
// hold E complex values in registers:
//   stage 1: thread t holds x[t + G*n1]; a radix-E DFT over n1 in registers, multiplication
//            by W_N^(t*k1), store to the group's LDS scratch;
//   barrier;
//   stage 2: thread t gathers, for each k1 = t + G*j, the G values of column k1, runs a
//            radix-G DFT in registers and ends up holding X[k1 + E*k2].
// This is the four-step (Bailey) decomposition with one LDS exchange per 1D transform.
//
// The 2D real transform of a (hin x win) plane placed at the origin of an (FH x FW) grid:
//   rows:    pairs of live rows are packed as (row_a + i*row_b) and transformed together;
//            rows >= hin are never touched (row pruning);
//   columns: the FW/2+1 half-spectrum columns; the two purely real columns (DC and Nyquist)
//            are packed into one complex column, so FW/2 column transforms cover all of them.
// The inverse runs the same steps backwards and only materialises the requested window of
// output rows (circularly offset, which gives both the overlap-save crop and the unshifted
// roll of the backward for free).
#pragma once

#include "nc_common.h"
#include "nc_twiddles.h"

template <int N>
struct FftShape;
template <>
struct FftShape<16> { static constexpr int E = 4, G = 4; };
template <>
struct FftShape<32> { static constexpr int E = 8, G = 4; };
template <>
struct FftShape<64> { static constexpr int E = 8, G = 8; };
template <>
struct FftShape<128> { static constexpr int E = 16, G = 8; };
template <>
struct FftShape<256> { static constexpr int E = 16, G = 16; };

// ---------------------------------------------------------------------------------------
// Register DFTs (natural-order in, natural-order out).  Forward: exp(-2*pi*i*n*k/N).
// ---------------------------------------------------------------------------------------

template <bool INV>
NC_DEV void dft4(cpx& a0, cpx& a1, cpx& a2, cpx& a3) {
    cpx s02 = cadd(a0, a2), d02 = csub(a0, a2);
    cpx s13 = cadd(a1, a3), d13 = csub(a1, a3);
    cpx r = INV ? cmul_i(d13) : cmul_negi(d13);
    a0 = cadd(s02, s13);
    a2 = csub(s02, s13);
    a1 = cadd(d02, r);
    a3 = csub(d02, r);
}

template <bool INV>
NC_DEV void dft8(cpx* v) {
    cpx e0 = v[0], e1 = v[2], e2 = v[4], e3 = v[6];
    cpx o0 = v[1], o1 = v[3], o2 = v[5], o3 = v[7];
    dft4<INV>(e0, e1, e2, e3);
    dft4<INV>(o0, o1, o2, o3);
    const float c = 0.70710678118654752f;
    o1 = cmul(o1, cmk(c, INV ? c : -c));
    o2 = INV ? cmul_i(o2) : cmul_negi(o2);
    o3 = cmul(o3, cmk(-c, INV ? c : -c));
    v[0] = cadd(e0, o0);
    v[4] = csub(e0, o0);
    v[1] = cadd(e1, o1);
    v[5] = csub(e1, o1);
    v[2] = cadd(e2, o2);
    v[6] = csub(e2, o2);
    v[3] = cadd(e3, o3);
    v[7] = csub(e3, o3);
}

// W_16^j, j = 0..9 (forward sign).
NC_DEV cpx w16(int j, bool inv) {
    const float c1 = 0.92387953251128674f, s1 = 0.38268343236508978f, c2 = 0.70710678118654752f;
    cpx w;
    switch (j) {
        case 0: w = cmk(1.f, 0.f); break;
        case 1: w = cmk(c1, -s1); break;
        case 2: w = cmk(c2, -c2); break;
        case 3: w = cmk(s1, -c1); break;
        case 4: w = cmk(0.f, -1.f); break;
        case 6: w = cmk(-c2, -c2); break;
        case 9: w = cmk(-c1, s1); break;
        default: w = cmk(1.f, 0.f); break;
    }
    if (inv) w.y = -w.y;
    return w;
}

template <bool INV>
NC_DEV void dft16(cpx* v) {
    cpx a[4][4];
#pragma unroll
    for (int n2 = 0; n2 < 4; ++n2) {
        a[n2][0] = v[n2];
        a[n2][1] = v[n2 + 4];
        a[n2][2] = v[n2 + 8];
        a[n2][3] = v[n2 + 12];
        dft4<INV>(a[n2][0], a[n2][1], a[n2][2], a[n2][3]);
    }
#pragma unroll
    for (int n2 = 1; n2 < 4; ++n2)
#pragma unroll
        for (int k1 = 1; k1 < 4; ++k1) a[n2][k1] = cmul(a[n2][k1], w16(n2 * k1, INV));
#pragma unroll
    for (int k1 = 0; k1 < 4; ++k1) {
        cpx b0 = a[0][k1], b1 = a[1][k1], b2 = a[2][k1], b3 = a[3][k1];
        dft4<INV>(b0, b1, b2, b3);
        v[k1] = b0;
        v[k1 + 4] = b1;
        v[k1 + 8] = b2;
        v[k1 + 12] = b3;
    }
}

template <int N, bool INV>
NC_DEV void dft_reg(cpx* v) {
    if constexpr (N == 4) {
        dft4<INV>(v[0], v[1], v[2], v[3]);
    } else if constexpr (N == 8) {
        dft8<INV>(v);
    } else {
        static_assert(N == 16, "radix");
        dft16<INV>(v);
    }
}

// W_N^e from the 256-point table (0 <= e < N); `tw` is the table's LDS copy.
template <int N, bool INV>
NC_DEV cpx twiddle(int e, const cpx* tw) {
    cpx w = tw[e * (256 / N)];
    if (INV) w.y = -w.y;
    return w;
}

// What a forward half-spectrum kernel applies to each bin before storing it:
//   kPostNone   the spectrum itself;
//   kPostAdd    plus add[kh][kw], one (FH, FW/2+1) spectrum shared by every plane;
//   kPostShift  times W_FH^(kh*sh) * W_FW^(kw*sw): the spectrum of the plane circularly
//               shifted by (sh, sw) on the grid (0 <= sh < FH, 0 <= sw < FW).
enum { kPostNone = 0, kPostAdd = 1, kPostShift = 2 };
struct SpecPost {
    const cpx* add;
    int sh, sw;
};

// W_FH^(kh*sh) * W_FW^(kw*sw), the phase ramp of a circular shift (exact table twiddles).
template <int FH, int FW>
NC_DEV cpx spec_ramp(int kh, int kw, int sh, int sw) {
    const float2 a = NC_TW256[((kh * sh) & (FH - 1)) * (NC_TW_N / FH)];
    const float2 b = NC_TW256[((kw * sw) & (FW - 1)) * (NC_TW_N / FW)];
    return cmul(cmk(a.x, a.y), cmk(b.x, b.y));
}

template <int POST, int FH, int FW>
NC_DEV cpx spec_post(cpx v, int kh, int kw, const SpecPost& p) {
    if constexpr (POST == kPostAdd) return cadd(v, p.add[kh * (FW / 2 + 1) + kw]);
    if constexpr (POST == kPostShift) return cmul(v, spec_ramp<FH, FW>(kh, kw, p.sh, p.sw));
    return v;
}

// Copies the twiddle table into LDS (256 cpx); callers barrier before first use.
NC_DEV void load_twiddles(cpx* tw) {
    for (int i = threadIdx.x; i < NC_TW_N; i += blockDim.x) tw[i] = NC_TW256[i];
}

// Cooperative, coalesced copy of an (h x w) row-major plane into LDS (as floats).
NC_DEV void stage_plane(const float* __restrict__ src, int n, float* dst) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = src[i];
}

// ---------------------------------------------------------------------------------------
// Group FFT stages (see file header).  scr: the group's LDS scratch, E*(G+1) cpx.
// ---------------------------------------------------------------------------------------

template <int N>
struct GroupFft {
    static constexpr int E = FftShape<N>::E;
    static constexpr int G = FftShape<N>::G;
    static constexpr int SCR = E * (G + 1);  // padded rows: fewer LDS bank conflicts
    static constexpr int J = E / G;          // column sets per thread in stage 2
    // Output slot s = j*G + k2 of thread t holds bin (t + G*j) + E*k2.
    static NC_DEV int bin(int t, int s) { return (t + G * (s / G)) + E * (s % G); }
};

template <int N, bool INV>
NC_DEV void gfft_stage1(cpx* v, int t, cpx* scr, const cpx* tw) {
    using F = GroupFft<N>;
    dft_reg<F::E, INV>(v);
#pragma unroll
    for (int k1 = 0; k1 < F::E; ++k1) {
        cpx y = v[k1];
        if (k1 > 0) y = cmul(y, twiddle<N, INV>(t * k1, tw));
        scr[k1 * (F::G + 1) + t] = y;
    }
}

template <int N, bool INV>
NC_DEV void gfft_stage2(cpx* v, int t, const cpx* scr) {
    using F = GroupFft<N>;
#pragma unroll
    for (int j = 0; j < F::J; ++j) {
        const int k1 = t + F::G * j;
        cpx u[F::G];
#pragma unroll
        for (int t2 = 0; t2 < F::G; ++t2) u[t2] = scr[k1 * (F::G + 1) + t2];
        dft_reg<F::G, INV>(u);
#pragma unroll
        for (int k2 = 0; k2 < F::G; ++k2) v[j * F::G + k2] = u[k2];
    }
}

// ---------------------------------------------------------------------------------------
// Plane geometry and LDS budget for an (FH x FW) spectral grid.
// ---------------------------------------------------------------------------------------

template <int FH, int FW>
struct Plane {
    static constexpr int SP = FW / 2 + 1;    // half-spectrum row pitch (cpx)
    static constexpr int F = FH * SP;        // half-spectrum size (cpx)
    using GH = GroupFft<FH>;
    using GW = GroupFft<FW>;
    static constexpr int NCG = FW / 2;       // column transforms (DC+Nyquist packed)
    static constexpr int NRG = FH / 2;       // max row-pair transforms
    static constexpr int TA = NRG * GW::G;   // threads to run every row pair at once
    static constexpr int TB = NCG * GH::G;   // threads to run every column at once
    static constexpr int NT0 = TA > TB ? TA : TB;
    static constexpr int NT = NT0 < 64 ? 64 : NT0;  // workgroup size (multiple of 64)
    static constexpr int WORK = (NRG * FW > FH * SP) ? NRG * FW : FH * SP;  // Zb / Tb (cpx)
    static constexpr int SCRA = (NT / GW::G) * GW::SCR;
    static constexpr int SCRB = (NT / GH::G) * GH::SCR;
    static constexpr int SCRN = SCRA > SCRB ? SCRA : SCRB;  // exchange scratch (cpx)
};

// Forward 2D real FFT of a (hin x win) real plane placed at the origin.
// load(r, c) is called only for r < hin, c < win.  Result: S[kh*SP + kw], kh < FH,
// kw <= FW/2.  Must be called by all NT threads (contains barriers; ends with one).
template <int FH, int FW, class Load>
NC_DEV void plane_rfft2(Load load, int hin, int win, cpx* S, cpx* Zb, cpx* scr,
                        const cpx* tw) {
    using P = Plane<FH, FW>;
    constexpr int EW = P::GW::E, GW = P::GW::G, EH = P::GH::E, GH = P::GH::G;
    constexpr int SP = P::SP;
    const int tid = threadIdx.x;

    // Phase A: packed row pairs -> Zb[p*FW + k], full FW complex bins.
    const int npairs = (hin + 1) >> 1;
    constexpr int GA = P::NT / GW;
    for (int p0 = 0; p0 < npairs; p0 += GA) {
        const int g = tid / GW, t = tid % GW, p = p0 + g;
        const bool on = p < npairs;
        cpx v[EW];
        if (on) {
            const int ra = 2 * p, rb = 2 * p + 1;
#pragma unroll
            for (int n1 = 0; n1 < EW; ++n1) {
                const int c = t + GW * n1;
                float a = 0.f, b = 0.f;
                if (c < win) {
                    a = load(ra, c);
                    if (rb < hin) b = load(rb, c);
                }
                v[n1] = cmk(a, b);
            }
            gfft_stage1<FW, false>(v, t, scr + g * P::GW::SCR, tw);
        }
        __syncthreads();
        if (on) {
            gfft_stage2<FW, false>(v, t, scr + g * P::GW::SCR);
#pragma unroll
            for (int s = 0; s < EW; ++s) Zb[p * FW + P::GW::bin(t, s)] = v[s];
        }
        __syncthreads();
    }

    // Phase B: column transforms over kh.  Group kw=0 packs (DC + i*Nyquist).
    constexpr int GB = P::NT / GH;
    for (int g0 = 0; g0 < P::NCG; g0 += GB) {
        const int g = tid / GH, t = tid % GH, kw = g0 + g;
        const bool on = kw < P::NCG;
        cpx v[EH];
        if (on) {
#pragma unroll
            for (int n1 = 0; n1 < EH; ++n1) {
                const int r = t + GH * n1;
                cpx val = cmk(0.f, 0.f);
                if (r < hin) {
                    const int p = r >> 1;
                    const bool odd = r & 1;
                    if (kw == 0) {
                        cpx z0 = Zb[p * FW], zn = Zb[p * FW + FW / 2];
                        val = odd ? cmk(z0.y, zn.y) : cmk(z0.x, zn.x);
                    } else {
                        cpx A = Zb[p * FW + kw];
                        cpx Bc = cconj(Zb[p * FW + FW - kw]);
                        val = odd ? cmul_negi(cscale(csub(A, Bc), 0.5f))
                                  : cscale(cadd(A, Bc), 0.5f);
                    }
                }
                v[n1] = val;
            }
            gfft_stage1<FH, false>(v, t, scr + g * P::GH::SCR, tw);
        }
        __syncthreads();
        if (on) {
            gfft_stage2<FH, false>(v, t, scr + g * P::GH::SCR);
            const int col = kw == 0 ? FW / 2 : kw;  // packed column parked in the Nyquist slot
#pragma unroll
            for (int s = 0; s < EH; ++s) S[P::GH::bin(t, s) * SP + col] = v[s];
        }
        __syncthreads();
    }

    // Unpack the packed column: C = P + iQ with P, Q spectra of real sequences.
    constexpr int UPT = (FH + P::NT - 1) / P::NT;
    cpx x0[UPT], xn[UPT];
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
        const int kh = tid + u * P::NT;
        if (kh < FH) {
            cpx c = S[kh * SP + FW / 2];
            cpx cm = cconj(S[((FH - kh) & (FH - 1)) * SP + FW / 2]);
            x0[u] = cscale(cadd(c, cm), 0.5f);
            xn[u] = cmul_negi(cscale(csub(c, cm), 0.5f));
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
        const int kh = tid + u * P::NT;
        if (kh < FH) {
            S[kh * SP] = x0[u];
            S[kh * SP + FW / 2] = xn[u];
        }
    }
    __syncthreads();
}

// Inverse 2D real FFT (unnormalised inverse times `scale`) of a half-spectrum supplied by
// spec(kh, kw) (kw <= FW/2), materialising only output rows r with
// i = (r - row0) mod FH < hout and columns c with j = (c - col0) mod FW < wout;
// store(i, j, value) receives them.  Tb: WORK cpx, scr: SCRN cpx.  All NT threads must call
// (contains barriers; ends with one).
template <int FH, int FW, class Spec, class Store>
NC_DEV void plane_irfft2(Spec spec, int row0, int hout, int col0, int wout, float scale,
                         Store store, cpx* Tb, cpx* scr, const cpx* tw) {
    using P = Plane<FH, FW>;
    constexpr int EW = P::GW::E, GW = P::GW::G, EH = P::GH::E, GH = P::GH::G;
    constexpr int SP = P::SP;
    const int tid = threadIdx.x;

    // Phase B': inverse column transforms, keeping only the requested rows.
    constexpr int GB = P::NT / GH;
    for (int g0 = 0; g0 < P::NCG; g0 += GB) {
        const int g = tid / GH, t = tid % GH, kw = g0 + g;
        const bool on = kw < P::NCG;
        cpx v[EH];
        if (on) {
#pragma unroll
            for (int n1 = 0; n1 < EH; ++n1) {
                const int kh = t + GH * n1;
                if (kw == 0) {
                    cpx a = spec(kh, 0), b = spec(kh, FW / 2);
                    v[n1] = cadd(a, cmul_i(b));
                } else {
                    v[n1] = spec(kh, kw);
                }
            }
            gfft_stage1<FH, true>(v, t, scr + g * P::GH::SCR, tw);
        }
        __syncthreads();
        if (on) {
            gfft_stage2<FH, true>(v, t, scr + g * P::GH::SCR);
#pragma unroll
            for (int s = 0; s < EH; ++s) {
                const int r = P::GH::bin(t, s);
                const int i = (r - row0) & (FH - 1);
                if (i < hout) {
                    if (kw == 0) {
                        Tb[i * SP] = cmk(v[s].x, 0.f);
                        Tb[i * SP + FW / 2] = cmk(v[s].y, 0.f);
                    } else {
                        Tb[i * SP + kw] = v[s];
                    }
                }
            }
        }
        __syncthreads();
    }

    // Phase A': inverse row transforms on packed pairs of output rows.
    const int npairs = (hout + 1) >> 1;
    constexpr int GA = P::NT / GW;
    for (int p0 = 0; p0 < npairs; p0 += GA) {
        const int g = tid / GW, t = tid % GW, p = p0 + g;
        const bool on = p < npairs;
        const int ia = 2 * p, ib = 2 * p + 1;
        const bool hasb = ib < hout;
        cpx v[EW];
        if (on) {
#pragma unroll
            for (int n1 = 0; n1 < EW; ++n1) {
                const int k = t + GW * n1;
                cpx a, b = cmk(0.f, 0.f);
                if (k <= FW / 2) {
                    a = Tb[ia * SP + k];
                    if (hasb) b = Tb[ib * SP + k];
                } else {
                    a = cconj(Tb[ia * SP + FW - k]);
                    if (hasb) b = cconj(Tb[ib * SP + FW - k]);
                }
                v[n1] = cadd(a, cmul_i(b));
            }
            gfft_stage1<FW, true>(v, t, scr + g * P::GW::SCR, tw);
        }
        __syncthreads();
        if (on) {
            gfft_stage2<FW, true>(v, t, scr + g * P::GW::SCR);
#pragma unroll
            for (int s = 0; s < EW; ++s) {
                const int c = P::GW::bin(t, s);
                const int j = (c - col0) & (FW - 1);
                if (j < wout) {
                    store(ia, j, v[s].x * scale);
                    if (hasb) store(ib, j, v[s].y * scale);
                }
            }
        }
        __syncthreads();
    }
}

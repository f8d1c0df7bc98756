// 64-point FFTs over groups of 8 lanes, and the 64 x 64 real plane transforms built on them.
//
// A 64-point transform is an 8 x 8 decomposition (X[k1 + 8 k2] = sum over n2 of
// W64^(n2 k1) W8^(n2 k2) sum over n1 of x[8 n1 + n2] W8^(n1 k1)): lane t of a group holds
// x[8 n1 + t] in v[n1], runs an 8-point DFT over n1 in registers, multiplies by W64^(t k1),
// exchanges through the group's 64-value LDS slot (an 8 x 8 transpose) and runs the second
// 8-point DFT, leaving X[t + 8 k2] in v[k2].  The 8 lanes of a group sit in one wavefront, so
// the exchange needs no workgroup barrier (a wavefront's LDS operations complete in order).
//
// A 256-thread workgroup (32 groups) transforms one 64 x 64 plane: the row pass puts two real
// rows into one complex transform (one group per row pair, only the live rows), the column
// pass gives each of the 32 groups one column, with the real DC and Nyquist columns packed
// into one complex column.  Compared with one transform per lane pair, a plane takes about a
// third of the instructions and four times as many wavefronts share the work.
#pragma once

#include "nc_fft.h"
#include "nc_twiddles.h"

namespace r8 {

constexpr int kNT = 256;       // threads per plane
constexpr int kGroups = 32;    // 8-lane groups per plane
// LDS pitches, chosen against bank conflicts.  The LDS serves 8-byte accesses 16 lanes (two
// groups) per pass over 16 bank pairs, a cpx at index a in pair a mod 16:
// - a group's exchange slot is 8 x 9 cpx and slots lie 72 cpx apart: the 8 x 8 transpose's
//   row writes (k1 * 9 + t) and column reads (t * 9 + n2) of two groups hit 16 pairs;
// - the row-transformed rows and the half-spectrum staging lie 34 cpx apart: the column
//   pass reads R[r * 34 + g] and writes O[kh * 34 + g] with r, kh = t + 8 * k (t = lane in
//   group), 2t + g distinct over the 16 lanes; the row pass's writes R[(2g + i) * 34 + k]
//   meet two lanes per pair (no pitch serves both patterns without a conflict).
constexpr int kEx = 72;        // cpx per group exchange slot (8 rows of 9)
constexpr int kXP = 9;         // exchange row pitch (cpx)
constexpr int kSP = 64 + 4;    // staging pitch (floats) of real rows
constexpr int kRP = 34;        // pitch (cpx) of the row-transformed rows (bins 0..32)
constexpr int kOP = 34;        // pitch (cpx) of the half-spectrum staging (bins 0..32)
constexpr int kF = 64 * 33;    // half-spectrum bins

// LDS layout of the forward plane transform (cpx units): the exchange slots, then one region
// shared in turn by the real input staging, the row-transformed rows and the output.
constexpr int kExCpx = kGroups * kEx;
constexpr int kMaxCpx(int a, int b) { return a > b ? a : b; }
constexpr int kRegionCpx = kMaxCpx(kMaxCpx(64 * kRP, 64 * kOP), 64 * kSP / 2);
constexpr size_t kFwdLdsBytes = (size_t)(kExCpx + kRegionCpx) * sizeof(cpx);

// Per-lane twiddles W64^(t k1), k1 = 0..7 (forward sign), from the 256-point table.
struct Tw {
    cpx w[8];
};

NC_DEV Tw twiddles(int t) {
    Tw r;
#pragma unroll
    for (int k1 = 0; k1 < 8; ++k1) r.w[k1] = NC_TW256[(4 * t * k1) & 255];
    return r;
}

// 64-point DFT of the group: in v[n1] = x[8 n1 + t], out v[k2] = X[t + 8 k2] (unnormalised;
// INV: inverse sign).  ex: the group's exchange slot.
template <bool INV>
NC_DEV void fft64(cpx* v, int t, const Tw& tw, cpx* ex) {
    dft8<INV>(v);
#pragma unroll
    for (int k1 = 1; k1 < 8; ++k1) v[k1] = cmul(v[k1], INV ? cconj(tw.w[k1]) : tw.w[k1]);
#pragma unroll
    for (int k1 = 0; k1 < 8; ++k1) ex[k1 * kXP + t] = v[k1];
    NC_WAVE_SYNC();
#pragma unroll
    for (int n2 = 0; n2 < 8; ++n2) v[n2] = ex[t * kXP + n2];
    NC_WAVE_SYNC();
    dft8<INV>(v);
}

// Forward real 2D transform of one (hin x win) plane at the origin of the 64 x 64 grid into
// the half-spectrum staging O (64 rows x kOP cpx, bins kw = 0..32), which aliases the input
// staging: on entry S (hin rows of kSP floats, columns win..63 zero) holds the plane.  All
// 256 threads call it; it starts and ends with a barrier.
NC_DEV void fwd_plane(float* lds, int hin, const Tw& tw) {
    cpx* exs = reinterpret_cast<cpx*>(lds);
    float* S = lds + 2 * kExCpx;
    cpx* R = reinterpret_cast<cpx*>(S);  // row-transformed rows: R[r * kRP + kw], kw <= 32
    cpx* O = R;                          // half-spectrum: O[kh * kOP + kw]
    const int tid = threadIdx.x, g = tid >> 3, t = tid & 7;
    cpx* ex = exs + g * kEx;
    const int npairs = (hin + 1) >> 1;
    __syncthreads();
    // row pass: group g transforms rows (2g, 2g + 1) as one complex row; wavefronts whose
    // groups are all past the live rows skip it (a wavefront-uniform branch), the others run
    // their idle groups on zeros without storing
    cpx v[8];
    const bool on = g < npairs, wave_on = 8 * (tid >> 6) < npairs;
    if (wave_on) {
        const int ga = on ? g : 0;
        const float* ra = S + 2 * ga * kSP;
        const float* rb = S + (2 * ga + 1 < hin ? 2 * ga + 1 : 2 * ga) * kSP;
        const float as = on ? 1.f : 0.f, bs = on && 2 * g + 1 < hin ? 1.f : 0.f;
#pragma unroll
        for (int n1 = 0; n1 < 8; ++n1) v[n1] = cmk(as * ra[8 * n1 + t], bs * rb[8 * n1 + t]);
    }
    __syncthreads();  // S is overwritten by R below
    if (wave_on) {
        fft64<false>(v, t, tw, ex);
        // split the two real rows: A[k] = (Z[k] + conj Z[-k]) / 2, B[k] = -i (Z[k] - conj Z[-k]) / 2
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) ex[t + 8 * k2] = v[k2];
        NC_WAVE_SYNC();
        cpx* ra = R + 2 * g * kRP;
        cpx* rb = R + (2 * g + 1) * kRP;
        const bool hb = 2 * g + 1 < hin;
#pragma unroll
        for (int k2 = 0; k2 < 5; ++k2) {
            const int k = t + 8 * k2;
            if (k <= 32 && on) {
                const cpx z = v[k2], m = ex[(64 - k) & 63];
                ra[k] = cmk(0.5f * (z.x + m.x), 0.5f * (z.y - m.y));
                if (hb) rb[k] = cmk(0.5f * (z.y + m.y), 0.5f * (m.x - z.x));
            }
        }
    }
    __syncthreads();
    // column pass: group g transforms column g; group 0 the packed column DC + i * Nyquist
#pragma unroll
    for (int n1 = 0; n1 < 8; ++n1) {
        const int r = 8 * n1 + t;
        cpx x = cmk(0.f, 0.f);
        if (r < hin) {
            const cpx* rr = R + r * kRP;
            x = g ? rr[g] : cmk(rr[0].x, rr[32].x);
        }
        v[n1] = x;
    }
    __syncthreads();  // R is overwritten by O below
    fft64<false>(v, t, tw, ex);
    if (tid < 64) {  // wavefront 0: group 0's unpack needs its bins' mirrors
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) ex[t + 8 * k2] = v[k2];
        NC_WAVE_SYNC();
    }
    if (g) {
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) O[(t + 8 * k2) * kOP + g] = v[k2];
    } else {
        // unpack DC (C0 = (P + conj P[-kh]) / 2) and Nyquist (C32 = -i (P - conj P[-kh]) / 2)
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) {
            const int kh = t + 8 * k2;
            const cpx p = v[k2], m = ex[(64 - kh) & 63];
            O[kh * kOP] = cmk(0.5f * (p.x + m.x), 0.5f * (p.y - m.y));
            O[kh * kOP + 32] = cmk(0.5f * (p.y + m.y), 0.5f * (m.x - p.x));
        }
    }
    __syncthreads();
}

}  // namespace r8

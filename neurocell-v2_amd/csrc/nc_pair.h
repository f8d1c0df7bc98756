// Lane-pair 2D real FFTs for (FH x FW) spectral grids with FH, FW in {32, 64}: one plane per
// 64-lane wavefront, every 1D transform over two adjacent lanes.
//
// A lane pair (lane = 2p + t) computes an N-point FFT by radix-2 decimation in time: lane t
// holds the N/2 samples x[2j + t], transforms them in registers (fft_reg), the odd lane applies
// W_N^k, and one DPP swap between the two lanes forms X[k] = E[k] + W^k O[k] on the even lane
// and X[k + N/2] = E[k] - W^k O[k] on the odd lane.  Compared with a whole N-point transform in
// one lane this halves the registers and the serial work per lane, so twice as many wavefronts
// (one per plane) are in flight.
//
//   column pass  pair p <-> packed column kc = p (FW/2 of them); rows kh = 2j + t in, rows
//                t*FH/2 + k out.  Column 0 carries DC + i*Nyquist, unpacked with its row mirror.
//   row pass     pair q <-> row pair (q, q + NR); columns 2j + t in, t*FW/2 + k out.  The
//                Hermitian split of the packed pair needs each bin's mirror, which sits in the
//                partner lane at slot N/2 - k: one DPP swap per bin.
//
// LDS: T holds the transposed half-spectrum rows (pitch FW/2 + 2 cpx).  The forward keeps the
// live rows plus a trash row and a zero row (as in nc_wave.h); the inverse keeps all FH rows so
// its stores have constant offsets, and the row pass applies the window's row offset (the
// windowed column pass, pcol_inv_rows, keeps only the window's rows with predicated stores,
// for kernels that trade those for a smaller LDS footprint).  The LDS serves 8-byte accesses
// 16 lanes per pass over 16 bank pairs (a cpx at index a in pair a mod 16): with the pitch
// even (2 mod 16) the row pass's reads of 8 consecutive rows by lane pairs (row, t) hit 16
// pairs, and the inverse's second row half starts kPairGap cpx further on, so the column
// pass's stores from the two lanes of a pair (rows k and FH/2 + k of column kc) land 8 pairs
// apart.
constexpr int kPairGap = 8;
#pragma once

#include "nc_wave.h"

// The value of v in the other lane of this lane's pair (DPP quad_perm [1,0,3,2]).
NC_DEV float pair_swap(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
NC_DEV cpx pair_swap(cpx v) { return cmk(pair_swap(v.x), pair_swap(v.y)); }

// N-point FFT over a lane pair (t = lane & 1): on entry lane t holds x[2j + t] in v[j]
// (j < N/2); on exit it holds X[t*N/2 + k] in v[k].  INV: inverse (unnormalised).
template <int N, bool INV>
NC_DEV void fft_pair(cpx* v, int t) {
    constexpr int H = N / 2;
    fft_reg<H, INV>(v);
    const float sg = t ? -1.f : 1.f;
#pragma unroll
    for (int k = 0; k < H; ++k) {
        cpx o = v[k];
        if (k > 0) {
            const cpx w = twm<N, INV>(o, k);
            o = t ? w : o;
        }
        const cpx r = pair_swap(o);
        v[k] = cmk(fmaf(sg, o.x, r.x), fmaf(sg, o.y, r.y));
    }
}

template <int FH, int FW>
struct PGeo {
    static_assert((FH == 32 || FH == 64) && FW == 64, "lane-pair grids");
    static constexpr int SP = FW / 2 + 1;  // half-spectrum row pitch (cpx)
    static constexpr int F = FH * SP;      // half-spectrum size (cpx)
    static constexpr int NC = FW / 2;      // packed columns = lane pairs of the column pass
    static constexpr int PITCH = NC + 2;   // LDS pitch of a transposed row (cpx)
    static constexpr int PF = FH * NC;     // packed spectrum size (cpx)
    static constexpr int HH = FH / 2;      // column samples per lane
    static constexpr int HW = FW / 2;      // row samples per lane
    // offset (cpx) of row r of the inverse's T: rows FH/2 .. FH-1 follow a kPairGap gap
    static NC_DEV int trow(int r) { return r * PITCH + (r >= HH ? kPairGap : 0); }
};

// The mirror partner of slot k for a spectrum held as lane t: bin t*N/2 + k.  The bin's mirror
// (N - bin) mod N is the partner lane's slot N/2 - k (k >= 1) or the bin itself (k == 0).
// Returns the mirror value of every slot of v in m (all lanes take part in the swaps).
template <int H>
NC_DEV void pair_mirror(const cpx* v, cpx* m) {
    m[0] = v[0];
#pragma unroll
    for (int k = 1; k < H; ++k) m[k] = pair_swap(v[H - k]);
}

// Forward row pass over the staged real rows S (rows x (FW + 1) floats, columns >= the plane
// width zero): row pairs (q, q + NR) -> packed half-spectrum rows of T (column 0 = DC +
// i*Nyquist), plus T's zero row.  All lanes must call it.  A barrier separates the reads of S
// from the stores, so S may share LDS with T.
template <int FH, int FW>
NC_DEV void prow_fwd(const float* S, int rows, cpx* T) {
    using P = PGeo<FH, FW>;
    const int lane = threadIdx.x & 63, q0 = lane >> 1, t = lane & 1;
    const int NR = (rows + 1) >> 1;
    const bool on = q0 < NR;
    const int q = on ? q0 : 0;
    const int rb = q + NR;
    const bool hb = on && rb < rows;
    const float* sa = S + q * (FW + 1);
    const float* sb = S + (hb ? rb : q) * (FW + 1);
    const float bs = hb ? 1.f : 0.f;
    cpx v[P::HW];
#pragma unroll
    for (int j = 0; j < P::HW; ++j) v[j] = cmk(sa[2 * j + t], sb[2 * j + t] * bs);
    fft_pair<FW, false>(v, t);
    cpx mr[P::HW];
    pair_mirror<P::HW>(v, mr);
    const cpx oth = pair_swap(v[0]);  // the partner's slot 0: Z(FW/2) on the even lane, Z(0) odd
    __syncthreads();
    // even lane: row a, bins k; odd lane: row b, bins HW - k (its own bins are their mirrors)
    const int trash = rows;
    cpx* ta = T + (on ? q : trash) * P::PITCH;
    cpx* tb = T + (hb ? rb : trash) * P::PITCH;
    // slot 0: DC and Nyquist of both rows are real; they are packed as DC + i*Nyquist
    if (t == 0) ta[0] = cmk(v[0].x, oth.x);
    else tb[0] = cmk(oth.y, v[0].y);
#pragma unroll
    for (int k = 1; k < P::HW; ++k) {
        const cpx own = v[k], r = mr[k];
        if (t == 0) ta[k] = cscale(cadd(own, cconj(r)), 0.5f);
        else tb[P::HW - k] = cmul_negi(cscale(csub(r, cconj(own)), 0.5f));
    }
    T[(rows + 1) * P::PITCH + (lane >> 1)] = cmk(0.f, 0.f);
}

// Forward column pass: lane pair kc reads packed column kc of T at rows 2j + t (rows >= `rows`
// read the zero row) and leaves its FH-point spectrum in v: slot k = row t*FH/2 + k.
template <int FH, int FW>
NC_DEV void pcol_fwd(const cpx* T, int rows, cpx* v) {
    using P = PGeo<FH, FW>;
    const int lane = threadIdx.x & 63, kc = lane >> 1, t = lane & 1;
    const cpx* tc = T + kc;
    int rl = rows;
    NC_PIN(rl);
#pragma unroll
    for (int j = 0; j < P::HH; ++j) {
        const int r = 2 * j + t;
        v[j] = tc[(r < rl ? r : rl + 1) * P::PITCH];
    }
    fft_pair<FH, false>(v, t);
}

// Inverse column pass: v holds lane pair kc's packed spectrum column at rows 2j + t; every
// output row r lands in T row r (at P::trow(r): FH x PITCH cpx plus the gap), so each store
// has a constant offset; the row pass applies the window's row offset.
template <int FH, int FW>
NC_DEV void pcol_inv(cpx* v, cpx* T) {
    using P = PGeo<FH, FW>;
    const int lane = threadIdx.x & 63, kc = lane >> 1, t = lane & 1;
    fft_pair<FH, true>(v, t);
    cpx* tc = T + P::trow(t * P::HH) + kc;
#pragma unroll
    for (int k = 0; k < P::HH; ++k) tc[k * P::PITCH] = v[k];
}

// Inverse column pass keeping only a window of output rows: row r lands in T row
// (r - row0) mod FH when that is below `rows`, and is dropped otherwise, so T holds `rows`
// rows (the row pass then reads them with row0 = 0).  The stores are predicated per element,
// but the LDS holds fewer rows, which leaves room for more workgroups per CU.
template <int FH, int FW>
NC_DEV void pcol_inv_rows(cpx* v, cpx* T, int row0, int rows) {
    using P = PGeo<FH, FW>;
    const int lane = threadIdx.x & 63, kc = lane >> 1, t = lane & 1;
    fft_pair<FH, true>(v, t);
#pragma unroll
    for (int k = 0; k < P::HH; ++k) {
        const int i = (t * P::HH + k - row0) & (FH - 1);
        if (i < rows) T[P::trow(i) + kc] = v[k];
    }
}

// Inverse row pass: output rows i < rows, taken from T row (i + row0) mod FH (packed
// half-spectrum rows), times scale, into the staging O (row i at O[i * (FW + 1)], every one of
// the FW columns stored at (c - col0) mod FW; row `rows` is the trash row).  All lanes must call
// it; a barrier separates the reads of T from the stores, so O may share LDS with T.
template <int FH, int FW>
NC_DEV void prow_inv(const cpx* T, int row0, int col0, int rows, float scale, float* O) {
    using P = PGeo<FH, FW>;
    const int lane = threadIdx.x & 63, q0 = lane >> 1, t = lane & 1;
    const int NR = (rows + 1) >> 1;
    const bool on = q0 < NR;
    const int q = on ? q0 : 0;
    const int ib = q + NR;
    const bool hb = on && ib < rows;
    const cpx* ta = T + P::trow((q + row0) & (FH - 1));
    const cpx* tb = T + P::trow(((hb ? ib : q) + row0) & (FH - 1));
    const float bs = hb ? 1.f : 0.f;
    cpx v[P::HW];
#pragma unroll
    for (int j = 0; j < P::HW; ++j) {
        cpx a, b;
        if (j == 0) {  // column t: the packed DC (even lane) or column 1
            const cpx a0 = ta[0], b0 = tb[0], a1 = ta[1], b1 = tb[1];
            a = t ? a1 : cmk(a0.x, 0.f);
            b = t ? b1 : cmk(b0.x, 0.f);
        } else if (j < P::HW / 2) {
            a = (ta + t)[2 * j];
            b = (tb + t)[2 * j];
        } else if (j == P::HW / 2) {  // column FW/2 + t: the packed Nyquist or conj(column FW/2 - 1)
            const cpx a0 = ta[0], b0 = tb[0], a1 = ta[P::HW - 1], b1 = tb[P::HW - 1];
            a = t ? cconj(a1) : cmk(a0.y, 0.f);
            b = t ? cconj(b1) : cmk(b0.y, 0.f);
        } else {
            a = cconj((ta - t)[FW - 2 * j]);
            b = cconj((tb - t)[FW - 2 * j]);
        }
        v[j] = cadd(a, cmul_i(cscale(b, bs)));
    }
    fft_pair<FW, true>(v, t);
    __syncthreads();
    float* oa = O + (on ? q : rows) * (FW + 1);
    float* ob = O + (hb ? ib : rows) * (FW + 1);
    int sh = t * P::HW + FW - col0;  // a vector copy, so the column offsets stay vector values
    NC_PIN(sh);
#pragma unroll
    for (int k = 0; k < P::HW; ++k) {
        const int jj = (k + sh) & (FW - 1);
        oa[jj] = v[k].x * scale;
        ob[jj] = v[k].y * scale;
    }
}

// Copies the staged output rows (rows x cols, row pitch FW + 1) to dst, contiguous: element
// e = i * cols + j per lane, all 64 lanes busy (i = floor(e / cols) by a 20-bit reciprocal,
// exact for e < 4096 and cols <= 64).
template <int FW>
NC_DEV void pstage_copy(const float* O, int rows, int cols, float* __restrict__ dst) {
    const int lane = threadIdx.x & 63;
    const int total = rows * cols;
    const unsigned inv = ((1u << 20) + cols - 1) / cols;
    constexpr int U = 8;
    for (int e0 = lane; e0 < total; e0 += 64 * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = min(e0 + 64 * u, total - 1);
            const int i = (int)(((unsigned)e * inv) >> 20);
            v[u] = O[i * (FW + 1) + (e - i * cols)];
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (e0 + 64 * u < total) dst[e0 + 64 * u] = v[u];
    }
}

// Half-spectrum store of a forward column pass: lane pair kc holds packed column kc at rows
// t*FH/2 + k.  Column 0 (DC + i*Nyquist) is split with its row mirrors; store(k, kh, kw, value)
// receives every bin of the half-spectrum (k: the register slot, kh = t*FH/2 + k).  All lanes
// take part in the swaps.
template <int FH, int FW, class Store>
NC_DEV void pstore_half(const cpx* v, Store store) {
    using P = PGeo<FH, FW>;
    const int lane = threadIdx.x & 63, kc = lane >> 1, t = lane & 1;
    cpx mr[P::HH];
    pair_mirror<P::HH>(v, mr);
    const int base = t * P::HH;
    if (kc != 0) {
#pragma unroll
        for (int k = 0; k < P::HH; ++k) store(k, base + k, kc, v[k]);
    } else {
#pragma unroll
        for (int k = 0; k < P::HH; ++k) {
            const cpx c = v[k], d = cconj(mr[k]);
            store(k, base + k, 0, cscale(cadd(c, d), 0.5f));
            store(k, base + k, FW / 2, cmul_negi(cscale(csub(c, d), 0.5f)));
        }
    }
}

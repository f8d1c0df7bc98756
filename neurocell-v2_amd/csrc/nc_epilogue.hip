// Piece 3: pure-ROI fused hidden-step epilogue and the output-port epilogue.
//
// Single pass (N = h*w <= 8192), one workgroup per sample b (kernels_pallas.py:163-291):
//   every thread owns PPT pixels of the plane for a chunk of MC directions in registers;
//   the MC plane sums (then the MC centred sums of squares) are reduced across the
//   workgroup at once (wave64 butterflies + a fixed-order cross-wave sum), so the two-pass
//   variance costs two block reductions per chunk, and z is read from HBM exactly once.
// Tiled (N > 8192), the (B, M, tiles) Chan parallel-variance pipeline
// (kernels_pallas.py:298-660): per-tile (s1, m2) -> exact Chan combine (recomputed by each
// consumer in fixed order) -> per-(b, tile) standardise + Codd + M-reduction.
// Output port (kernels_pallas.py:1076-1551): plane statistics, standardisation of the P
// port cells only, and a backward whose sparse port scatter is applied in registers through
// an LDS pixel->slot map, one workgroup per (b, tile).
// B-reductions (gw/gs/gb, gdb, port parameters) are fixed-order column sums: no atomics.
#include <algorithm>
#include <mutex>

#include "nc_common.h"
#include "nc_large.h"

namespace {

constexpr int kSingleMaxPix = 8192;  // kernels_pallas.py:56
constexpr int kTileN = 1024;         // kernels_pallas.py:58
constexpr int kPortTile = 2048;
constexpr int kMaxM = 64;

// 16-byte loads and stores need 16-byte aligned planes.
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The border term z + hb * delta is read branch-free: with hb == 0 the kernels read z's own
// (cached) pixels through `dl` and scale them by 0.  A uniform `if (hb)` inside the unrolled
// element loops would make the compiler wait for every element's loads before issuing the
// next ones, serialising the whole plane.
NC_DEV const float* border_src(int hb, const float* delta, const float* z) {
    return hb ? delta : z;
}

// t[q][k] = z[zi(q, k)] (+ delta[di(q, k)] when hb) for an MC x PPT register tile: the two
// forms are whole unrolled loops behind one uniform branch, so either issues all its loads
// together, and without the border term z is read once.
template <int MC, int PPT, class ZI, class DI>
NC_DEV void load_tile(float (&t)[MC][PPT], int hb, const float* __restrict__ z,
                      const float* __restrict__ delta, ZI zi, DI di) {
    if (hb) {
#pragma unroll
        for (int q = 0; q < MC; ++q)
#pragma unroll
            for (int k = 0; k < PPT; ++k) t[q][k] = z[zi(q, k)] + delta[di(q, k)];
    } else {
#pragma unroll
        for (int q = 0; q < MC; ++q)
#pragma unroll
            for (int k = 0; k < PPT; ++k) t[q][k] = z[zi(q, k)];
    }
}

// ----------------------------------------------------------------------------------------
// Single pass (N <= 8192): grid (B, G).  Workgroup (b, g) owns sample b's directions
// [g * mpg, min(M, (g + 1) * mpg)), processed in chunks of MC held in registers.  With
// G == 1 one workgroup owns the whole sample; at small batches the directions are split
// over G workgroups so that every CU has work, and their partial sums over directions are
// added in fixed order by a second launch (k_group_sum / k_port_combine): the kernel boundary
// makes every XCD's partials visible without device-scope fences inside the kernel.
// ----------------------------------------------------------------------------------------

template <int NT, int PPT, int MC, int ACT>
__global__ __launch_bounds__(NT) void k_epi_fwd(int M, int N, int mpg, float slope, int hb,
                                                const float* __restrict__ z,
                                                const float* __restrict__ delta,
                                                const float* __restrict__ w,
                                                const float* __restrict__ s,
                                                const float* __restrict__ bb,
                                                float* __restrict__ out, float* __restrict__ mean,
                                                float* __restrict__ rstd,
                                                float* __restrict__ part) {
    __shared__ float red[MC * (NT / 64) + MC];
    const int b = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int B = gridDim.x, G = gridDim.y;
    const int mb = g * mpg, me = min(M, mb + mpg);
    const float inv_n = 1.0f / (float)N;
    float lin[PPT], ac[PPT], bv[PPT], wv[PPT], sv[PPT];
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
        const int pc = min(tid + k * NT, N - 1);
        lin[k] = 0.f;
        ac[k] = 0.f;
        bv[k] = bb[pc];
        wv[k] = w[pc];
        sv[k] = s[pc];
    }
    for (int m0 = mb; m0 < me; m0 += MC) {
        float zt[MC][PPT];
        float sum[MC];
        // unconditional (clamped) loads keep all MC*PPT requests in flight together
        load_tile<MC, PPT>(
            zt, hb, z, delta,
            [&](int q, int k) {
                return ((size_t)b * M + min(m0 + q, me - 1)) * N + min(tid + k * NT, N - 1);
            },
            [&](int q, int k) {
                return (size_t)min(m0 + q, me - 1) * N + min(tid + k * NT, N - 1);
            });
#pragma unroll
        for (int q = 0; q < MC; ++q) sum[q] = 0.f;
#pragma unroll
        for (int q = 0; q < MC; ++q)
#pragma unroll
            for (int k = 0; k < PPT; ++k)
                sum[q] += (m0 + q < me && tid + k * NT < N) ? zt[q][k] : 0.f;
        block_sum<MC, NT>(sum, red);
        float mu[MC], sq[MC];
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            mu[q] = sum[q] * inv_n;
            sq[q] = 0.f;
#pragma unroll
            for (int k = 0; k < PPT; ++k) {
                const float d = tid + k * NT < N ? zt[q][k] - mu[q] : 0.f;
                sq[q] += d * d;
            }
        }
        block_sum<MC, NT>(sq, red);
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            const int m = m0 + q;
            if (m >= me) break;
            const float r = 1.0f / sqrtf(sq[q] * inv_n + 1e-5f);
#pragma unroll
            for (int k = 0; k < PPT; ++k) {
                const float zn = (zt[q][k] - mu[q]) * r;
                lin[k] += zn;
                ac[k] += act_f<ACT>(zn + bv[k], slope);
            }
            if (tid == 0) {
                mean[(size_t)b * M + m] = mu[q];
                rstd[(size_t)b * M + m] = r;
            }
        }
    }
    float* dst = G == 1 ? out + (size_t)b * N : part + ((size_t)g * B + b) * N;
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
        const int p = tid + k * NT;
        if (p < N) dst[p] = wv[k] * lin[k] + sv[k] * ac[k];
    }
}

// out[i] = sum over g < G of part[g * n + i], fixed order (the split forward's combine).
__global__ __launch_bounds__(256) void k_group_sum(int G, size_t n, const float* __restrict__ part,
                                                   float* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float acc = part[i];
    for (int q = 1; q < G; ++q) acc += part[(size_t)q * n + i];
    out[i] = acc;
}

// Backward: gz of the workgroup's directions and its partial gw/gs/gb over them, written as
// row (g, b) of pg (3, G*B, N) and reduced over all G*B rows afterwards.
//
// The workgroup's directions run in register chunks of MC, software-pipelined: the next
// chunk's planes are loaded before the current chunk's arithmetic, block reduction and gz
// stores (its barriers wait for LDS only, so the loads stay in flight), and the chunks
// alternate between two register tiles.  With VEC (N % 4 == 0, PPT a multiple of 4) a thread
// owns runs of 4 consecutive pixels, moved as 16-byte loads and stores.
template <int NT, int PPT, bool VEC>
struct EpiPix {
    // pixel of register slot k
    static NC_DEV int at(int tid, int k) {
        if constexpr (VEC) return 4 * (tid + (k >> 2) * NT) + (k & 3);
        else return tid + k * NT;
    }
};

// t[q][k] = z (+ delta) of plane row `zrow(q)` (delta row `drow(q)`) at the thread's pixels,
// clamped to the plane; all loads issue together.
template <int NT, int PPT, int MC, bool VEC, class ZR, class DR>
NC_DEV void load_chunk(float (&t)[MC][PPT], int hb, int N, const float* __restrict__ z,
                       const float* __restrict__ delta, int tid, ZR zrow, DR drow) {
    if constexpr (VEC) {
        const int nv = N >> 2;
        if (hb) {
#pragma unroll
            for (int q = 0; q < MC; ++q) {
                const float4* zp = reinterpret_cast<const float4*>(z + zrow(q));
                const float4* dp = reinterpret_cast<const float4*>(delta + drow(q));
#pragma unroll
                for (int j = 0; j < PPT / 4; ++j) {
                    const int v = min(tid + j * NT, nv - 1);
                    const float4 a = zp[v], d = dp[v];
                    t[q][4 * j] = a.x + d.x;
                    t[q][4 * j + 1] = a.y + d.y;
                    t[q][4 * j + 2] = a.z + d.z;
                    t[q][4 * j + 3] = a.w + d.w;
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < MC; ++q) {
                const float4* zp = reinterpret_cast<const float4*>(z + zrow(q));
#pragma unroll
                for (int j = 0; j < PPT / 4; ++j) {
                    const float4 a = zp[min(tid + j * NT, nv - 1)];
                    t[q][4 * j] = a.x;
                    t[q][4 * j + 1] = a.y;
                    t[q][4 * j + 2] = a.z;
                    t[q][4 * j + 3] = a.w;
                }
            }
        }
    } else {
        load_tile<MC, PPT>(
            t, hb, z, delta, [&](int q, int k) { return zrow(q) + min(tid + k * NT, N - 1); },
            [&](int q, int k) { return drow(q) + min(tid + k * NT, N - 1); });
    }
}

template <int NT, int PPT, int MC, int ACT, bool VEC>
__global__ __launch_bounds__(NT) void k_epi_bwd(
    int M, int N, int mpg, float slope, int hb, const float* __restrict__ z,
    const float* __restrict__ delta, const float* __restrict__ w, const float* __restrict__ s,
    const float* __restrict__ bb, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gy, float* __restrict__ gz, float* __restrict__ pg, size_t GBN) {
    using Px = EpiPix<NT, PPT, VEC>;
    __shared__ float red[2 * MC * (NT / 64) + 2 * MC];
    const int b = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int mb = g * mpg, me = min(M, mb + mpg);
    const float inv_n = 1.0f / (float)N;
    auto zrow = [&](int m0) {
        return [=](int q) { return ((size_t)b * M + min(m0 + q, me - 1)) * N; };
    };
    auto drow = [&](int m0) { return [=](int q) { return (size_t)min(m0 + q, me - 1) * N; }; };
    float ta[MC][PPT], tb[MC][PPT];
    load_chunk<NT, PPT, MC, VEC>(ta, hb, N, z, delta, tid, zrow(mb), drow(mb));
    float lin[PPT], ac[PPT], dbs[PPT], bv[PPT], wv[PPT], sv[PPT], gv[PPT];
    if constexpr (VEC) {  // runs of 4 pixels: one 16-byte load per operand
        const int nv = N >> 2;
#pragma unroll
        for (int j = 0; j < PPT / 4; ++j) {
            const int v = min(tid + j * NT, nv - 1);
            const bool in = tid + j * NT < nv;
            const float4 b4 = reinterpret_cast<const float4*>(bb)[v];
            const float4 w4 = reinterpret_cast<const float4*>(w)[v];
            const float4 s4 = reinterpret_cast<const float4*>(s)[v];
            const float4 g4 = reinterpret_cast<const float4*>(gy + (size_t)b * N)[v];
            const float bq[4] = {b4.x, b4.y, b4.z, b4.w}, wq[4] = {w4.x, w4.y, w4.z, w4.w};
            const float sq[4] = {s4.x, s4.y, s4.z, s4.w}, gq[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int k = 4 * j + u;
                lin[k] = ac[k] = dbs[k] = 0.f;
                bv[k] = bq[u];
                wv[k] = wq[u];
                sv[k] = sq[u];
                gv[k] = in ? gq[u] : 0.f;  // zero cotangent outside the plane
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < PPT; ++k) {
            const int pc = min(Px::at(tid, k), N - 1);
            lin[k] = ac[k] = dbs[k] = 0.f;
            bv[k] = bb[pc];
            wv[k] = w[pc];
            sv[k] = s[pc];
            const float gl = gy[(size_t)b * N + pc];
            gv[k] = Px::at(tid, k) < N ? gl : 0.f;  // zero cotangent outside the plane
        }
    }
    // one chunk: its arithmetic on `cur` with the next chunk's loads into `nxt` in flight
    auto chunk = [&](float (&cur)[MC][PPT], float (&nxt)[MC][PPT], int m0) {
        if (m0 + MC < me)
            load_chunk<NT, PPT, MC, VEC>(nxt, hb, N, z, delta, tid, zrow(m0 + MC),
                                         drow(m0 + MC));
        float c[2 * MC], mr[MC], rr[MC], gzn[MC][PPT];
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            const int m = min(m0 + q, me - 1);
            mr[q] = mean[(size_t)b * M + m];
            rr[q] = rstd[(size_t)b * M + m];
        }
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            const bool mv = m0 + q < me;
            c[q] = c[MC + q] = 0.f;
#pragma unroll
            for (int k = 0; k < PPT; ++k) {
                const float nz = (cur[q][k] - mr[q]) * rr[q];
                float a;
                const float da = act_fd<ACT>(nz + bv[k], slope, &a);
                const float gn = mv ? gv[k] * (wv[k] + sv[k] * da) : 0.f;
                if (mv) {
                    lin[k] += nz;
                    ac[k] += a;
                    dbs[k] += sv[k] * gv[k] * da;
                }
                cur[q][k] = nz;
                gzn[q][k] = gn;
                c[q] += gn;
                c[MC + q] += gn * nz;
            }
        }
        block_sum<2 * MC, NT>(c, red);
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            const int m = m0 + q;
            if (m >= me) break;
            const float c1 = c[q] * inv_n, c2 = c[MC + q] * inv_n;
            float o[PPT];
#pragma unroll
            for (int k = 0; k < PPT; ++k) o[k] = rr[q] * (gzn[q][k] - c1 - cur[q][k] * c2);
            float* dst = gz + ((size_t)b * M + m) * N;
            if constexpr (VEC) {
#pragma unroll
                for (int j = 0; j < PPT / 4; ++j) {
                    const int v = tid + j * NT;
                    if (4 * v < N)
                        reinterpret_cast<float4*>(dst)[v] =
                            make_float4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
                }
            } else {
#pragma unroll
                for (int k = 0; k < PPT; ++k) {
                    const int p = tid + k * NT;
                    if (p < N) dst[p] = o[k];
                }
            }
        }
    };
    for (int m0 = mb; m0 < me; m0 += 2 * MC) {
        chunk(ta, tb, m0);
        if (m0 + MC < me) chunk(tb, ta, m0 + MC);
    }
    const size_t row = ((size_t)g * gridDim.x + b) * N;  // GBN: the gw / gs / gb plane stride
    float o0[PPT], o1[PPT];
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
        o0[k] = gv[k] * lin[k];
        o1[k] = gv[k] * ac[k];
    }
    const bool pg_vec = ((reinterpret_cast<uintptr_t>(pg + row) | (GBN * 4)) & 15) == 0;
    if (VEC && pg_vec) {
#pragma unroll
        for (int j = 0; j < PPT / 4; ++j) {
            const int v = tid + j * NT;
            if (4 * v < N) {
                float4* p0 = reinterpret_cast<float4*>(pg + row);
                float4* p1 = reinterpret_cast<float4*>(pg + GBN + row);
                float4* p2 = reinterpret_cast<float4*>(pg + 2 * GBN + row);
                p0[v] = make_float4(o0[4 * j], o0[4 * j + 1], o0[4 * j + 2], o0[4 * j + 3]);
                p1[v] = make_float4(o1[4 * j], o1[4 * j + 1], o1[4 * j + 2], o1[4 * j + 3]);
                p2[v] = make_float4(dbs[4 * j], dbs[4 * j + 1], dbs[4 * j + 2], dbs[4 * j + 3]);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < PPT; ++k) {
            const int p = Px::at(tid, k);
            if (p < N) {
                pg[row + p] = o0[k];
                pg[GBN + row + p] = o1[k];
                pg[2 * GBN + row + p] = dbs[k];
            }
        }
    }
}

// Fixed-order sums over rows, several independent jobs per launch (blockIdx.y = job):
// job.out[x] = (job.acc ? job.out[x] : 0) + sum over r < job.rows of job.in[r * job.X + x].
// A job with no input and no rows writes zeros (a cotangent that is identically zero).
// A workgroup's Q = blockDim.x / 64 waves form Q / qs column groups of 64 columns; the qs
// waves of a group (qs from the job's row count, about 32 rows per wave) sum fixed contiguous
// slices of its rows (coalesced) and the qs slice sums are added in fixed order, so the
// result is deterministic for given shapes.
constexpr int kRedParts = 16;
constexpr int kRedJobs = 10;

struct RedJob {
    const float* in;
    float* out;
    int X;
    int acc;
    int rows;  // number of rows summed (the batch, or groups x batch)
    int qs;    // waves per column group (set at launch)
};

struct RedJobs {
    RedJob j[kRedJobs];
};

__global__ __launch_bounds__(64 * kRedParts) void k_batch_reduce(RedJobs jobs) {
    __shared__ float part[kRedParts][64];
    const RedJob J = jobs.j[blockIdx.y];
    const int B = J.rows;
    const int Q = blockDim.x >> 6, qs = J.qs, cols = (Q / qs) * 64;
    if ((int)blockIdx.x * cols >= J.X) return;  // uniform over the workgroup
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, q = w % qs;
    const int x = blockIdx.x * cols + (w / qs) * 64 + lane;
    const int b0 = (B * q) / qs, b1 = (B * (q + 1)) / qs;
    float s = 0.f;
    if (x < J.X && b1 > b0) {
        const float* src = J.in + x;
        float a[4] = {0.f, 0.f, 0.f, 0.f};
        int b = b0;
        for (; b + 4 <= b1; b += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) a[u] += src[(size_t)(b + u) * J.X];
        }
        for (; b < b1; ++b) a[0] += src[(size_t)b * J.X];
        s = (a[0] + a[1]) + (a[2] + a[3]);
    }
    part[w][lane] = s;
    __syncthreads();
    if (q == 0 && x < J.X) {
        float t = 0.f;
        for (int k = 0; k < qs; ++k) t += part[w + k][lane];
        float* o = J.out + x;
        *o = J.acc ? *o + t : t;
    }
}

// Launches the non-empty jobs of `jobs` (in order) as one k_batch_reduce.
int launch_batch_reduce(hipStream_t st, const RedJob* jobs, int njobs) {
    RedJobs pack{};
    int n = 0, rmax = 0;
    auto slices = [](int rows) {  // about 32 rows per wave, 1..16 waves
        int q = 1;
        while (q < kRedParts && q * 32 < rows) q *= 2;
        return q;
    };
    for (int i = 0; i < njobs; ++i) {
        if (!jobs[i].out || jobs[i].X <= 0 || (!jobs[i].in && jobs[i].rows > 0)) continue;
        pack.j[n++] = jobs[i];
        rmax = std::max(rmax, jobs[i].rows);
    }
    if (n == 0) return NC_OK;
    const int Q = slices(rmax);
    int nblk = 0;
    for (int i = 0; i < n; ++i) {
        pack.j[i].qs = slices(pack.j[i].rows);
        const int cols = (Q / pack.j[i].qs) * 64;
        nblk = std::max(nblk, (pack.j[i].X + cols - 1) / cols);
    }
    hipLaunchKernelGGL(k_batch_reduce, dim3(nblk, n), dim3(64 * Q), 0, st, pack);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

// ----------------------------------------------------------------------------------------
// Tiled (Chan) pipeline for N > 8192.
// ----------------------------------------------------------------------------------------

constexpr int kTileNT = 256;
constexpr int kTilePPT = kTileN / kTileNT;

// A thread's kTilePPT pixels of a tile: with VEC four consecutive pixels, moved as one 16-byte
// access per plane (N % 4 == 0, so every tile holds a multiple of 4 pixels), otherwise pixels
// kTileNT apart.  Loads are clamped into the tile; `in` says which pixels are real.
static_assert(kTilePPT == 4, "one 16-byte access per plane and thread");

template <bool VEC>
struct TilePx {
    static NC_DEV bool in(int tid, int k, int nt) {
        return VEC ? 4 * tid < nt : tid + k * kTileNT < nt;
    }
    // p: the plane's tile base
    static NC_DEV void load(const float* __restrict__ p, int tid, int nt,
                            float (&v)[kTilePPT]) {
        if constexpr (VEC) {
            const float4 a = reinterpret_cast<const float4*>(p)[min(tid, (nt >> 2) - 1)];
            v[0] = a.x;
            v[1] = a.y;
            v[2] = a.z;
            v[3] = a.w;
        } else {
#pragma unroll
            for (int k = 0; k < kTilePPT; ++k) v[k] = p[min(tid + k * kTileNT, nt - 1)];
        }
    }
    // the real pixels only; 16-byte stores when p is 16-byte aligned (a uniform test)
    static NC_DEV void store(float* __restrict__ p, int tid, int nt,
                             const float (&v)[kTilePPT]) {
        if (VEC && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
            if (4 * tid < nt)
                reinterpret_cast<float4*>(p)[tid] = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int k = 0; k < kTilePPT; ++k) {
                const int i = VEC ? 4 * tid + k : tid + k * kTileNT;
                if (i < nt) p[i] = v[k];
            }
        }
    }
};

// 16-byte accesses apply when every plane the tiled kernels read that way is 16-byte aligned
// (the pixel mapping, and so the reduction order, then depends on the inputs only).
inline bool tile_vec(int N, int hb, const float* z, const float* delta, const float* w,
                     const float* s, const float* bb, const float* gy = nullptr) {
    return N % 4 == 0 && aligned16(z) && (!hb || aligned16(delta)) && aligned16(w) &&
           aligned16(s) && aligned16(bb) && (!gy || aligned16(gy));
}

// Per-(b, m, tile) sum and centred sum of squares; stats layout (2, B, M, T).
template <bool VEC>
__global__ __launch_bounds__(kTileNT) void k_tile_stats(int M, int N, int T, int hb,
                                                        const float* __restrict__ z,
                                                        const float* __restrict__ delta,
                                                        float* __restrict__ stats) {
    using Px = TilePx<VEC>;
    __shared__ float red[kTileNT / 64 + 1];
    const int t = blockIdx.x, m = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
    const int base = t * kTileN;
    const int nt = min(kTileN, N - base);
    const float* zp = z + ((size_t)b * M + m) * N + base;
    const float* dp = border_src(hb, delta + (size_t)m * N, z + ((size_t)b * M + m) * N) + base;
    const float hbf = hb ? 1.f : 0.f;
    float v[kTilePPT], d[kTilePPT];
    Px::load(zp, tid, nt, v);
    Px::load(dp, tid, nt, d);
    float s1 = 0.f;
#pragma unroll
    for (int k = 0; k < kTilePPT; ++k) {
        v[k] = Px::in(tid, k, nt) ? v[k] + hbf * d[k] : 0.f;
        s1 += v[k];
    }
    block_sum<1, kTileNT>(&s1, red);
    const float mu = s1 / (float)nt;
    float m2 = 0.f;
#pragma unroll
    for (int k = 0; k < kTilePPT; ++k) {
        const float dv = Px::in(tid, k, nt) ? v[k] - mu : 0.f;
        m2 += dv * dv;
    }
    block_sum<1, kTileNT>(&m2, red);
    if (tid == 0) {
        const size_t BMT = (size_t)gridDim.z * M * T;
        const size_t o = ((size_t)b * M + m) * T + t;
        stats[o] = s1;
        stats[BMT + o] = m2;
    }
}

void tile_stats(hipStream_t st, bool vec, int B, int M, int N, int T, int hb, const float* z,
                const float* delta, float* stats) {
    if (vec)
        hipLaunchKernelGGL(k_tile_stats<true>, dim3(T, M, B), dim3(kTileNT), 0, st, M, N, T, hb,
                           z, delta, stats);
    else
        hipLaunchKernelGGL(k_tile_stats<false>, dim3(T, M, B), dim3(kTileNT), 0, st, M, N, T, hb,
                           z, delta, stats);
}

// Chan combine of the T tile statistics of plane (b, m) by one wavefront: each lane takes
// tiles lane, lane + 64, ... in order, then a butterfly over the lanes (fixed order).  Every
// lane returns the result.  Tiles hold tn consecutive pixels, the last one the rest.
NC_DEV void chan_combine_wave(const float* stats, size_t BMT, int b, int m, int M, int N, int T,
                              int tn, float* mean, float* rstd) {
    const int lane = threadIdx.x & (NC_WAVE - 1);
    const float* s1 = stats + ((size_t)b * M + m) * T;
    const float* m2 = s1 + BMT;
    float tot = 0.f;
    for (int t = lane; t < T; t += NC_WAVE) tot += s1[t];
    const float mu = wave_sum(tot) / (float)N;
    float var = 0.f;
    for (int t = lane; t < T; t += NC_WAVE) {
        const int nt = min(tn, N - t * tn);
        const float d = s1[t] / (float)nt - mu;
        var += m2[t] + (float)nt * d * d;
    }
    *mean = mu;
    *rstd = 1.0f / sqrtf(wave_sum(var) / (float)N + 1e-5f);
}

// Directions whose loads a tiled kernel keeps in flight together.
constexpr int kTileMC = 4;

// Per-(tile, b): statistics from the Chan partials (Ts tiles of tn pixels per plane), then
// standardise + Codd + sum over M.
template <int ACT, bool VEC>
__global__ __launch_bounds__(kTileNT) void k_tile_fwd(int B, int M, int N, int Ts, int tn,
                                                      float slope, int hb,
                                                      const float* __restrict__ z,
                                                      const float* __restrict__ delta,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ s,
                                                      const float* __restrict__ bb,
                                                      const float* __restrict__ stats,
                                                      float* __restrict__ out,
                                                      float* __restrict__ mean,
                                                      float* __restrict__ rstd) {
    using Px = TilePx<VEC>;
    __shared__ float smu[kMaxM], srs[kMaxM];
    const int t = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const size_t BMT = (size_t)B * M * Ts;
    // one wavefront per direction combines its tile statistics
    for (int m = tid / NC_WAVE; m < M; m += kTileNT / NC_WAVE) {
        float mu, r;
        chan_combine_wave(stats, BMT, b, m, M, N, Ts, tn, &mu, &r);
        if ((tid & (NC_WAVE - 1)) == 0) {
            smu[m] = mu;
            srs[m] = r;
            if (t == 0) {
                mean[(size_t)b * M + m] = mu;
                rstd[(size_t)b * M + m] = r;
            }
        }
    }
    const int base = t * kTileN;
    const int nt = min(kTileN, N - base);
    const float* dl = border_src(hb, delta, z);
    const float hbf = hb ? 1.f : 0.f;
    float lin[kTilePPT], ac[kTilePPT], bv[kTilePPT], wv[kTilePPT], sv[kTilePPT];
    Px::load(bb + base, tid, nt, bv);
    Px::load(w + base, tid, nt, wv);
    Px::load(s + base, tid, nt, sv);
#pragma unroll
    for (int k = 0; k < kTilePPT; ++k) lin[k] = ac[k] = 0.f;
    __syncthreads();
    for (int m0 = 0; m0 < M; m0 += kTileMC) {
        float v[kTileMC][kTilePPT], d[kTileMC][kTilePPT];
#pragma unroll
        for (int q = 0; q < kTileMC; ++q) {
            const int m = min(m0 + q, M - 1);
            Px::load(z + ((size_t)b * M + m) * N + base, tid, nt, v[q]);
            Px::load(dl + (size_t)m * N + base, tid, nt, d[q]);
        }
#pragma unroll
        for (int q = 0; q < kTileMC; ++q) {
            if (m0 + q >= M) break;
            const float mu = smu[m0 + q], r = srs[m0 + q];
#pragma unroll
            for (int k = 0; k < kTilePPT; ++k) {
                const float zn = (v[q][k] + hbf * d[q][k] - mu) * r;
                lin[k] += zn;
                ac[k] += act_f<ACT>(zn + bv[k], slope);
            }
        }
    }
    float o[kTilePPT];
#pragma unroll
    for (int k = 0; k < kTilePPT; ++k) o[k] = wv[k] * lin[k] + sv[k] * ac[k];
    Px::store(out + (size_t)b * N + base, tid, nt, o);
}

// Backward stage 1 per (tile, b): per-tile partial c1/c2 (layout (2, B, M, T)) and the
// per-sample gw/gs/gb partials pg (3, B, N).
template <int ACT, bool VEC>
__global__ __launch_bounds__(kTileNT) void k_tile_bwd1(
    int B, int M, int N, int T, float slope, int hb, const float* __restrict__ z,
    const float* __restrict__ delta, const float* __restrict__ w, const float* __restrict__ s,
    const float* __restrict__ bb, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gy, float* __restrict__ cpart, float* __restrict__ pg, size_t BN) {
    using Px = TilePx<VEC>;
    // per-wavefront (c1, c2) sums of every direction, red[wave][c1 | c2][m], added over the
    // wavefronts once after the direction loop
    constexpr int NWV = kTileNT / 64;
    __shared__ float red[NWV * 2 * kMaxM];
    const int t = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int base = t * kTileN;
    const int nt = min(kTileN, N - base);
    const float* dl = border_src(hb, delta, z);
    const float hbf = hb ? 1.f : 0.f;
    float lin[kTilePPT], ac[kTilePPT], dbs[kTilePPT], g[kTilePPT], wv[kTilePPT], sv[kTilePPT],
        bv[kTilePPT];
    Px::load(gy + (size_t)b * N + base, tid, nt, g);
    Px::load(w + base, tid, nt, wv);
    Px::load(s + base, tid, nt, sv);
    Px::load(bb + base, tid, nt, bv);
#pragma unroll
    for (int k = 0; k < kTilePPT; ++k) {
        lin[k] = ac[k] = dbs[k] = 0.f;
        if (!Px::in(tid, k, nt)) g[k] = 0.f;  // zero cotangent outside the tile
    }
    const size_t BMT = (size_t)B * M * T;
    for (int m0 = 0; m0 < M; m0 += kTileMC) {
        float v[kTileMC][kTilePPT], d[kTileMC][kTilePPT], mu[kTileMC], r[kTileMC],
            c[2 * kTileMC];
#pragma unroll
        for (int q = 0; q < kTileMC; ++q) {
            const int m = min(m0 + q, M - 1);
            mu[q] = mean[(size_t)b * M + m];
            r[q] = rstd[(size_t)b * M + m];
            Px::load(z + ((size_t)b * M + m) * N + base, tid, nt, v[q]);
            Px::load(dl + (size_t)m * N + base, tid, nt, d[q]);
        }
#pragma unroll
        for (int q = 0; q < kTileMC; ++q) {
            const bool mv = m0 + q < M;
            c[q] = c[kTileMC + q] = 0.f;
#pragma unroll
            for (int k = 0; k < kTilePPT; ++k) {
                const float zn = (v[q][k] + hbf * d[q][k] - mu[q]) * r[q];
                float a;
                const float da = act_fd<ACT>(zn + bv[k], slope, &a);
                const float gn = mv ? g[k] * (wv[k] + sv[k] * da) : 0.f;
                if (mv) {
                    lin[k] += zn;
                    ac[k] += a;
                    dbs[k] += sv[k] * g[k] * da;
                }
                c[q] += gn;
                c[kTileMC + q] += gn * zn;
            }
        }
        // wavefront sums now (no barrier), the workgroup sum after the loop
#pragma unroll
        for (int q = 0; q < kTileMC; ++q) {
            const float a1 = wave_sum(c[q]), a2 = wave_sum(c[kTileMC + q]);
            if (lane == 0 && m0 + q < M) {
                red[wave * 2 * kMaxM + m0 + q] = a1;
                red[wave * 2 * kMaxM + kMaxM + m0 + q] = a2;
            }
        }
    }
    __syncthreads();
    for (int e = tid; e < 2 * M; e += kTileNT) {
        const int k = e / M, m = e - k * M;  // k: c1 or c2
        float v = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < NWV; ++w2) v += red[w2 * 2 * kMaxM + k * kMaxM + m];
        cpart[(size_t)k * BMT + ((size_t)b * M + m) * T + t] = v;
    }
    float o0[kTilePPT], o1[kTilePPT];
#pragma unroll
    for (int k = 0; k < kTilePPT; ++k) {
        o0[k] = g[k] * lin[k];
        o1[k] = g[k] * ac[k];
    }
    float* p = pg + (size_t)b * N + base;  // BN: the gw / gs / gb plane stride
    Px::store(p, tid, nt, o0);
    Px::store(p + BN, tid, nt, o1);
    Px::store(p + 2 * BN, tid, nt, dbs);
}

// Backward stage 2 per (tile, m, b): gz = rstd * (gzn - c1 - zn * c2).
template <int ACT, bool VEC>
__global__ __launch_bounds__(kTileNT) void k_tile_bwd2(
    int B, int M, int N, int T, float slope, int hb, const float* __restrict__ z,
    const float* __restrict__ delta, const float* __restrict__ w, const float* __restrict__ s,
    const float* __restrict__ bb, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gy, const float* __restrict__ cpart, float* __restrict__ gz) {
    using Px = TilePx<VEC>;
    const int t = blockIdx.x, m = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
    const size_t BMT = (size_t)B * M * T;
    const float* c1p = cpart + ((size_t)b * M + m) * T;
    const float* c2p = c1p + BMT;
    const int base = t * kTileN;
    const int nt = min(kTileN, N - base);
    const float* zp = z + ((size_t)b * M + m) * N;
    const float* dp = border_src(hb, delta + (size_t)m * N, zp);
    const float hbf = hb ? 1.f : 0.f;
    float v[kTilePPT], d[kTilePPT], bv[kTilePPT], g[kTilePPT], wv[kTilePPT], sv[kTilePPT];
    Px::load(zp + base, tid, nt, v);
    Px::load(dp + base, tid, nt, d);
    Px::load(bb + base, tid, nt, bv);
    Px::load(gy + (size_t)b * N + base, tid, nt, g);
    Px::load(w + base, tid, nt, wv);
    Px::load(s + base, tid, nt, sv);
    // the plane's (c1, c2): the T tile partials summed by the workgroup (fixed order)
    __shared__ float red[2 * (kTileNT / 64) + 2];
    float c[2] = {0.f, 0.f};
    for (int u = tid; u < T; u += kTileNT) {
        c[0] += c1p[u];
        c[1] += c2p[u];
    }
    block_sum<2, kTileNT>(c, red);
    const float c1 = c[0] / (float)N, c2 = c[1] / (float)N;
    const float mu = mean[(size_t)b * M + m], r = rstd[(size_t)b * M + m];
    float o[kTilePPT];
#pragma unroll
    for (int k = 0; k < kTilePPT; ++k) {
        const float zn = (v[k] + hbf * d[k] - mu) * r;
        float a;
        const float da = act_fd<ACT>(zn + bv[k], slope, &a);
        const float gn = g[k] * (wv[k] + sv[k] * da);
        o[k] = r * (gn - c1 - zn * c2);
    }
    Px::store(gz + ((size_t)b * M + m) * N + base, tid, nt, o);
}

// ----------------------------------------------------------------------------------------
// Output port.
// ----------------------------------------------------------------------------------------

// Single-pass plane statistics of sample b's directions [mb, me) into LDS (N <= 8192).
template <int NT, int PPT, int MC>
NC_DEV void plane_stats(int b, int M, int mb, int me, int N, int hb, const float* __restrict__ z,
                        const float* __restrict__ delta, float* smu, float* srs, float* red) {
    const int tid = threadIdx.x;
    const float inv_n = 1.0f / (float)N;
    for (int m0 = mb; m0 < me; m0 += MC) {
        float zt[MC][PPT], sum[MC], sq[MC];
        load_tile<MC, PPT>(
            zt, hb, z, delta,
            [&](int q, int k) {
                return ((size_t)b * M + min(m0 + q, me - 1)) * N + min(tid + k * NT, N - 1);
            },
            [&](int q, int k) {
                return (size_t)min(m0 + q, me - 1) * N + min(tid + k * NT, N - 1);
            });
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            sum[q] = 0.f;
#pragma unroll
            for (int k = 0; k < PPT; ++k) {
                if (m0 + q >= me || tid + k * NT >= N) zt[q][k] = 0.f;
                sum[q] += zt[q][k];
            }
        }
        block_sum<MC, NT>(sum, red);
#pragma unroll
        for (int q = 0; q < MC; ++q) {
            sq[q] = 0.f;
            const float mu = sum[q] * inv_n;
#pragma unroll
            for (int k = 0; k < PPT; ++k) {
                const int p = tid + k * NT;
                const float d = p < N ? zt[q][k] - mu : 0.f;
                sq[q] += d * d;
            }
        }
        block_sum<MC, NT>(sq, red);
        if (tid == 0) {
#pragma unroll
            for (int q = 0; q < MC; ++q)
                if (m0 + q < me) {
                    smu[m0 + q] = sum[q] * inv_n;
                    srs[m0 + q] = 1.0f / sqrtf(sq[q] * inv_n + 1e-5f);
                }
        }
    }
    __syncthreads();
}

// Port algebra of one output cell from its direction sums (epilogue.py:82-128): lin = sum of
// the standardised port values, ac = sum of act(value + b_out).
NC_DEV float port_out(int M, int fact, float slope, float wo, float so, float bo, float lin,
                      float ac, float* pre) {
    if (fact == NC_ACT_IDENTITY) return (wo + so) * lin + (float)M * so * bo;
    const float y = wo * lin + so * ac;
    *pre = y;
    return nc_act(y, fact, slope);
}

// Gather + port algebra for sample b's directions [mb, me) once smu/srs are known.  With G > 1
// the direction sums go to part (2, G, B, P) and k_port_combine finishes the algebra.
NC_DEV void port_gather(int b, int B, int M, int mb, int me, int G, int g, int N, int P, int hb,
                        int fact, float slope, const int* __restrict__ pidx,
                        const float* __restrict__ z, const float* __restrict__ delta,
                        const float* __restrict__ pp, const float* smu, const float* srs,
                        float* szo, float* __restrict__ out, float* __restrict__ zo,
                        float* __restrict__ pre, float* __restrict__ part) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const int nm = me - mb;
    for (int q = tid; q < nm * P; q += nt) {
        const int m = mb + q / P, k = q % P;
        const int e = pidx[k];
        const float v = z[((size_t)b * M + m) * N + e] + (hb ? delta[(size_t)m * N + e] : 0.f);
        const float zn = (v - smu[m]) * srs[m];
        szo[q] = zn;
        zo[((size_t)b * M + m) * P + k] = zn;
    }
    if (!pp) return;  // standardisation only (uniform across the block)
    __syncthreads();
    const size_t GBP = (size_t)G * B * P;
    for (int k = tid; k < P; k += nt) {
        const float bo = pp[2 * P + k];
        float lin = 0.f, ac = 0.f;
        for (int m = 0; m < nm; ++m) {
            const float v = szo[m * P + k];
            lin += v;
            if (fact != NC_ACT_IDENTITY) ac += nc_act(v + bo, fact, slope);
        }
        if (G == 1) {
            out[(size_t)b * P + k] =
                port_out(M, fact, slope, pp[k], pp[P + k], bo, lin, ac, pre + (size_t)b * P + k);
        } else {
            part[((size_t)g * B + b) * P + k] = lin;
            part[GBP + ((size_t)g * B + b) * P + k] = ac;
        }
    }
}

// The split port forward's combine: direction sums over the G partials (fixed order), then the
// port algebra; one thread per (b, k).
__global__ __launch_bounds__(256) void k_port_combine(int B, int M, int P, int G, int fact,
                                                      float slope, const float* __restrict__ pp,
                                                      const float* __restrict__ part,
                                                      float* __restrict__ out,
                                                      float* __restrict__ pre) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= B * P) return;
    const int k = i % P;
    const size_t GBP = (size_t)G * B * P;
    float lin = 0.f, ac = 0.f;
    for (int q = 0; q < G; ++q) {
        lin += part[(size_t)q * B * P + i];
        ac += part[GBP + (size_t)q * B * P + i];
    }
    out[i] = port_out(M, fact, slope, pp[k], pp[P + k], pp[2 * P + k], lin, ac, pre + i);
}

template <int NT, int PPT, int MC>
__global__ __launch_bounds__(NT) void k_port_fwd(int M, int N, int mpg, int P, int hb, int fact,
                                                 float slope, const int* __restrict__ pidx,
                                                 const float* __restrict__ z,
                                                 const float* __restrict__ delta,
                                                 const float* __restrict__ pp,
                                                 float* __restrict__ out, float* __restrict__ zo,
                                                 float* __restrict__ mean,
                                                 float* __restrict__ rstd,
                                                 float* __restrict__ pre,
                                                 float* __restrict__ part) {
    HIP_DYNAMIC_SHARED(float, szo)  // mpg*P
    __shared__ float smu[kMaxM], srs[kMaxM];
    __shared__ float red[MC * (NT / 64) + MC];
    const int b = blockIdx.x, g = blockIdx.y;
    const int mb = g * mpg, me = min(M, mb + mpg);
    plane_stats<NT, PPT, MC>(b, M, mb, me, N, hb, z, delta, smu, srs, red);
    for (int m = mb + (int)threadIdx.x; m < me; m += NT) {
        mean[(size_t)b * M + m] = smu[m];
        rstd[(size_t)b * M + m] = srs[m];
    }
    port_gather(b, gridDim.x, M, mb, me, gridDim.y, g, N, P, hb, fact, slope, pidx, z, delta, pp,
                smu, srs, szo, out, zo, pre, part);
}

// Large planes: Chan partials (k_tile_stats) -> per-sample combine + gather.
__global__ __launch_bounds__(256) void k_port_fwd_tiled(
    int B, int M, int N, int T, int P, int hb, int fact, float slope,
    const int* __restrict__ pidx, const float* __restrict__ z, const float* __restrict__ delta,
    const float* __restrict__ pp, const float* __restrict__ stats, float* __restrict__ out,
    float* __restrict__ zo, float* __restrict__ mean, float* __restrict__ rstd,
    float* __restrict__ pre) {
    HIP_DYNAMIC_SHARED(float, szo)
    __shared__ float smu[kMaxM], srs[kMaxM];
    const int b = blockIdx.x;
    const size_t BMT = (size_t)B * M * T;
    for (int m = threadIdx.x / NC_WAVE; m < M; m += blockDim.x / NC_WAVE) {
        float mu, r;
        chan_combine_wave(stats, BMT, b, m, M, N, T, kTileN, &mu, &r);
        if ((threadIdx.x & (NC_WAVE - 1)) == 0) {
            smu[m] = mu;
            srs[m] = r;
            mean[(size_t)b * M + m] = mu;
            rstd[(size_t)b * M + m] = r;
        }
    }
    __syncthreads();
    port_gather(b, B, M, 0, M, 1, 0, N, P, hb, fact, slope, pidx, z, delta, pp, smu, srs, szo,
                out, zo, pre, nullptr);
}

// Port backward per (tile, direction group, b): port cotangents and (c1, c2) of every
// direction (cheap, recomputed by each workgroup), then the dense gz of the group's
// kPortMC directions over the tile with the sparse port term added in registers through an
// LDS pixel->slot map.  Workgroup (0, 0, b) also writes the per-sample port-parameter
// partials ppart (3, B, P).
constexpr int kPortNT = 256;
constexpr int kPortPPT = kPortTile / kPortNT;
constexpr int kPortMC = 4;

template <bool VEC>
__global__ __launch_bounds__(kPortNT) void k_port_bwd(
    int M, int N, int P, int hb, int fact, float slope, const int* __restrict__ pidx,
    const float* __restrict__ z, const float* __restrict__ delta, const float* __restrict__ pp,
    const float* __restrict__ zo, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ pre, const float* __restrict__ gout, float* __restrict__ gz,
    float* __restrict__ ppart, size_t pstride) {
    HIP_DYNAMIC_SHARED(float, dyn)
    float* gzo = dyn;                          // M*P: port cotangent per (m, k)
    float* gsum = dyn + M * P;                 // M*P: summed per first-occurrence slot
    float* zos = dyn + 2 * M * P;              // M*P: this sample's standardised port values
    int* slot = reinterpret_cast<int*>(dyn + 3 * M * P);  // kPortTile
    __shared__ float c1s[kMaxM], c2s[kMaxM];
    __shared__ int first[256];
    const int t = blockIdx.x, mg = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
    const float* zob = zo + (size_t)b * M * P;
    const int base = t * kPortTile;
    const int ntile = min(kPortTile, N - base);
    const int m0 = mg * kPortMC;
    // 0. the dense tile's loads first: they depend on nothing below, so their latency hides
    //    the port bookkeeping (thread pixels: strided, or runs of 4 with VEC)
    auto pix = [&](int k) {
        return VEC ? 4 * (tid + (k >> 2) * kPortNT) + (k & 3) : tid + k * kPortNT;
    };
    float v[kPortMC][kPortPPT];
    load_chunk<kPortNT, kPortPPT, kPortMC, VEC>(
        v, hb, ntile, z + base, delta + (hb ? base : 0), tid,
        [&](int q) { return ((size_t)b * M + min(m0 + q, M - 1)) * N; },
        [&](int q) { return (size_t)min(m0 + q, M - 1) * N; });
    // 1. port cotangents (given directly as (B,M,P) in standardisation-only mode)
    for (int q = tid; q < M * P; q += kPortNT) {
        gsum[q] = 0.f;
        const float zq = zob[q];
        zos[q] = zq;
        if (!pp) {
            gzo[q] = gout[(size_t)b * M * P + q];
            continue;
        }
        const int k = q % P;
        const float wo = pp[k], so = pp[P + k], bo = pp[2 * P + k];
        const float go = gout[(size_t)b * P + k];
        float val;
        if (fact == NC_ACT_IDENTITY) {
            val = go * (wo + so);
        } else {
            float a;
            const float gp = go * nc_act_d(pre[(size_t)b * P + k], fact, slope, &a);
            val = gp * (wo + so * nc_act_d(zq + bo, fact, slope, &a));
        }
        gzo[q] = val;
    }
    for (int i = tid; i < ntile; i += kPortNT) slot[i] = -1;
    __syncthreads();
    // 2. first-occurrence slots of the port cells inside this tile (sequential: duplicates
    //    of a coordinate port add up, as the reference's .at[].add does)
    if (tid == 0) {
        for (int k = 0; k < P; ++k) {
            const int e = pidx[k] - base;
            int f = -1;
            if (e >= 0 && e < ntile) {
                if (slot[e] < 0) slot[e] = k;
                f = slot[e];
            }
            first[k] = f;
        }
    }
    __syncthreads();
    for (int m = tid; m < M; m += kPortNT) {
        float a1 = 0.f, a2 = 0.f;
        for (int k = 0; k < P; ++k) {
            const float g = gzo[m * P + k];
            a1 += g;
            a2 += g * zos[m * P + k];
            if (first[k] >= 0) gsum[m * P + first[k]] += g;
        }
        c1s[m] = a1 / (float)N;
        c2s[m] = a2 / (float)N;
    }
    __syncthreads();
    // 3. dense gz of this group's directions over the tile
    int sl[kPortPPT];
#pragma unroll
    for (int k = 0; k < kPortPPT; ++k) sl[k] = slot[min(pix(k), ntile - 1)];
#pragma unroll
    for (int q = 0; q < kPortMC; ++q) {
        const int m = m0 + q;
        if (m >= M) break;
        const float mu = mean[(size_t)b * M + m], r = rstd[(size_t)b * M + m];
        const float c1 = c1s[m], c2 = c2s[m];
        float o[kPortPPT];
#pragma unroll
        for (int k = 0; k < kPortPPT; ++k) {
            const float zn = (v[q][k] - mu) * r;
            float gv = -r * (c1 + zn * c2);
            if (sl[k] >= 0) gv += r * gsum[m * P + sl[k]];
            o[k] = gv;
        }
        float* dst = gz + ((size_t)b * M + m) * N + base;
        if constexpr (VEC) {
#pragma unroll
            for (int j = 0; j < kPortPPT / 4; ++j) {
                const int vv = tid + j * kPortNT;
                if (4 * vv < ntile)
                    reinterpret_cast<float4*>(dst)[vv] =
                        make_float4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
            }
        } else {
#pragma unroll
            for (int k = 0; k < kPortPPT; ++k)
                if (tid + k * kPortNT < ntile) dst[tid + k * kPortNT] = o[k];
        }
    }
    // 4. per-sample port-parameter partials
    if (t == 0 && mg == 0 && pp) {
        for (int k = tid; k < P; k += kPortNT) {
            const float so = pp[P + k], bo = pp[2 * P + k];
            const float go = gout[(size_t)b * P + k];
            float lin = 0.f, ac = 0.f, gbv = 0.f;
            float gp = go;
            if (fact != NC_ACT_IDENTITY) {
                float a;
                gp = go * nc_act_d(pre[(size_t)b * P + k], fact, slope, &a);
            }
            for (int m = 0; m < M; ++m) {
                const float v2 = zob[m * P + k];
                lin += v2;
                if (fact != NC_ACT_IDENTITY) {
                    float a;
                    const float da = nc_act_d(v2 + bo, fact, slope, &a);
                    ac += a;
                    gbv += gp * so * da;
                }
            }
            float gw, gs, gb;
            if (fact == NC_ACT_IDENTITY) {
                gw = gp * lin;
                gs = gp * (lin + (float)M * bo);
                gb = gp * (float)M * so;
            } else {
                gw = gp * lin;
                gs = gp * ac;
                gb = gbv;
            }
            ppart[(size_t)b * P + k] = gw;  // pstride: the three parameters' plane stride
            ppart[pstride + (size_t)b * P + k] = gs;
            ppart[2 * pstride + (size_t)b * P + k] = gb;
        }
    }
}

// ----------------------------------------------------------------------------------------
// Launch configuration
// ----------------------------------------------------------------------------------------

struct SingleCfg {
    int nt, ppt;
};

SingleCfg single_cfg(int N) {
    if (N <= 256) return {256, 1};
    if (N <= 512) return {256, 2};
    if (N <= 768) return {256, 3};
    if (N <= 1024) return {256, 4};
    if (N <= 2048) return {512, 4};
    if (N <= 4096) return {1024, 4};
    return {1024, 8};
}

int tiles_of(int N) { return (N + kTileN - 1) / kTileN; }

// Direction split of the single-pass kernels.  Every thread keeps MC directions of its PPT
// pixels in registers (the backward two such tiles: zhat and its cotangent), all loaded
// together; MC shrinks as the workgroup grows so a thread stays within its VGPR share.  Below
// kWideBatch samples one workgroup per sample leaves CUs idle, so the directions are split
// over G workgroups of one MC chunk each (kSplitMC in the forward).
constexpr int kWideBatch = 512;
constexpr int kSplitMC = 4;

struct DirPlan {
    SingleCfg c;
    int mc;   // directions per register chunk
    int G;    // workgroups per sample
    int mpg;  // directions per workgroup
};

DirPlan fwd_plan(int B, int M, int N) {
    const SingleCfg c = single_cfg(N);
    const int whole = c.nt <= 512 ? 16 : (c.ppt == 4 ? 8 : 4);
    if (B >= kWideBatch || M <= kSplitMC) return {c, whole, 1, M};
    return {c, kSplitMC, (M + kSplitMC - 1) / kSplitMC, kSplitMC};
}

DirPlan bwd_plan(int B, int M, int N) {
    const SingleCfg c = single_cfg(N);
    const int mc = c.nt <= 512 ? 8 : (c.ppt == 4 ? 4 : 2);
    if (B >= kWideBatch || M <= mc || c.nt > 512) return {c, mc, 1, M};
    return {c, mc, (M + mc - 1) / mc, mc};
}

// Workspace carve-up (floats, each region 256-byte aligned).
struct EpiWs {
    float* pg;        // (3, Gb*B, N) per-(group, sample) gw/gs/gb partials
    float* stats;     // (4, B, M, T) tile statistics / backward (c1, c2) partials
    float* pport;     // (3, B, 256) port-parameter partials
    float* fpart;     // (Gf, B, N) forward partial outputs
    float* portpart;  // (2, Gf, B, 256) port forward partial direction sums
    size_t bytes;
};

EpiWs epi_ws(void* ws, int B, int M, int N) {
    const bool single = N <= kSingleMaxPix;
    const size_t Gf = single ? fwd_plan(B, M, N).G : 1;
    const size_t Gb = single ? bwd_plan(B, M, N).G : 1;
    const size_t T = tiles_of(N);
    float* base = reinterpret_cast<float*>(ws);
    size_t off = 0;
    auto take = [&](size_t n) {
        float* p = base ? base + off : nullptr;
        off += (n + 63) / 64 * 64;
        return p;
    };
    EpiWs e;
    e.pg = take(3 * Gb * B * N);
    e.stats = take(4 * (size_t)B * M * T);
    e.pport = take(3 * (size_t)B * 256);
    e.fpart = take(Gf * B * N);
    e.portpart = take(2 * Gf * B * 256);
    e.bytes = off * sizeof(float);
    return e;
}

#define NC_LAUNCH_ACT(KER, NT_, PPT_, MC_, ...) \
    hipLaunchKernelGGL((KER<NT_, PPT_, MC_, ACT>), __VA_ARGS__)

// Forward-side dispatch over (NT, PPT, MC) of a DirPlan.
#define NC_FWD_DISPATCH(P_, KER, ...)                                                           \
    do {                                                                                        \
        const SingleCfg c_ = P_.c;                                                              \
        const bool w_ = P_.mc != kSplitMC;                                                      \
        if (c_.nt == 256 && c_.ppt == 1) {                                                      \
            if (w_) NC_LAUNCH_ACT(KER, 256, 1, 16, __VA_ARGS__);                                \
            else NC_LAUNCH_ACT(KER, 256, 1, kSplitMC, __VA_ARGS__);                             \
        } else if (c_.nt == 256 && c_.ppt == 2) {                                               \
            if (w_) NC_LAUNCH_ACT(KER, 256, 2, 16, __VA_ARGS__);                                \
            else NC_LAUNCH_ACT(KER, 256, 2, kSplitMC, __VA_ARGS__);                             \
        } else if (c_.nt == 256 && c_.ppt == 3) {                                               \
            if (w_) NC_LAUNCH_ACT(KER, 256, 3, 16, __VA_ARGS__);                                \
            else NC_LAUNCH_ACT(KER, 256, 3, kSplitMC, __VA_ARGS__);                             \
        } else if (c_.nt == 256 && c_.ppt == 4) {                                               \
            if (w_) NC_LAUNCH_ACT(KER, 256, 4, 16, __VA_ARGS__);                                \
            else NC_LAUNCH_ACT(KER, 256, 4, kSplitMC, __VA_ARGS__);                             \
        } else if (c_.nt == 512) {                                                              \
            if (w_) NC_LAUNCH_ACT(KER, 512, 4, 16, __VA_ARGS__);                                \
            else NC_LAUNCH_ACT(KER, 512, 4, kSplitMC, __VA_ARGS__);                             \
        } else if (c_.ppt == 4) {                                                               \
            if (w_) NC_LAUNCH_ACT(KER, 1024, 4, 8, __VA_ARGS__);                                \
            else NC_LAUNCH_ACT(KER, 1024, 4, kSplitMC, __VA_ARGS__);                            \
        } else {                                                                                \
            NC_LAUNCH_ACT(KER, 1024, 8, 4, __VA_ARGS__);                                        \
        }                                                                                       \
    } while (0)

#define NC_LAUNCH_BWD(NT_, PPT_, MC_, VEC_, ...) \
    hipLaunchKernelGGL((k_epi_bwd<NT_, PPT_, MC_, ACT, VEC_>), __VA_ARGS__)
// Backward dispatch: register chunks of half the plan's group size (two or more pipelined
// chunks per workgroup), 16-byte pixel runs when N % 4 == 0 and PPT is a multiple of 4.
#define NC_BWD_DISPATCH(P_, VEC_OK, ...)                                                        \
    do {                                                                                        \
        const SingleCfg c_ = P_.c;                                                              \
        const bool v_ = (VEC_OK);                                                               \
        if (c_.nt == 256 && c_.ppt == 1) NC_LAUNCH_BWD(256, 1, 4, false, __VA_ARGS__);          \
        else if (c_.nt == 256 && c_.ppt == 2) NC_LAUNCH_BWD(256, 2, 4, false, __VA_ARGS__);     \
        else if (c_.nt == 256 && c_.ppt == 3) NC_LAUNCH_BWD(256, 3, 4, false, __VA_ARGS__);     \
        else if (c_.nt == 256 && c_.ppt == 4) {                                                 \
            if (v_) NC_LAUNCH_BWD(256, 4, 4, true, __VA_ARGS__);                                \
            else NC_LAUNCH_BWD(256, 4, 4, false, __VA_ARGS__);                                  \
        } else if (c_.nt == 512) {                                                              \
            if (v_) NC_LAUNCH_BWD(512, 4, 4, true, __VA_ARGS__);                                \
            else NC_LAUNCH_BWD(512, 4, 4, false, __VA_ARGS__);                                  \
        } else if (c_.ppt == 4) {                                                               \
            if (v_) NC_LAUNCH_BWD(1024, 4, 2, true, __VA_ARGS__);                               \
            else NC_LAUNCH_BWD(1024, 4, 2, false, __VA_ARGS__);                                 \
        } else {                                                                                \
            if (v_) NC_LAUNCH_BWD(1024, 8, 1, true, __VA_ARGS__);                               \
            else NC_LAUNCH_BWD(1024, 8, 1, false, __VA_ARGS__);                                 \
        }                                                                                       \
    } while (0)

// The port forward has no per-pixel activation.
#define NC_LAUNCH_PORT(NT_, PPT_, MC_, ...) hipLaunchKernelGGL((k_port_fwd<NT_, PPT_, MC_>), __VA_ARGS__)
#define NC_PORT_DISPATCH(P_, ...)                                                               \
    do {                                                                                        \
        const SingleCfg c_ = P_.c;                                                              \
        const bool w_ = P_.mc != kSplitMC;                                                      \
        if (c_.nt == 256 && c_.ppt == 1) {                                                      \
            if (w_) NC_LAUNCH_PORT(256, 1, 16, __VA_ARGS__);                                    \
            else NC_LAUNCH_PORT(256, 1, kSplitMC, __VA_ARGS__);                                 \
        } else if (c_.nt == 256 && c_.ppt == 2) {                                               \
            if (w_) NC_LAUNCH_PORT(256, 2, 16, __VA_ARGS__);                                    \
            else NC_LAUNCH_PORT(256, 2, kSplitMC, __VA_ARGS__);                                 \
        } else if (c_.nt == 256 && c_.ppt == 3) {                                               \
            if (w_) NC_LAUNCH_PORT(256, 3, 16, __VA_ARGS__);                                    \
            else NC_LAUNCH_PORT(256, 3, kSplitMC, __VA_ARGS__);                                 \
        } else if (c_.nt == 256 && c_.ppt == 4) {                                               \
            if (w_) NC_LAUNCH_PORT(256, 4, 16, __VA_ARGS__);                                    \
            else NC_LAUNCH_PORT(256, 4, kSplitMC, __VA_ARGS__);                                 \
        } else if (c_.nt == 512) {                                                              \
            if (w_) NC_LAUNCH_PORT(512, 4, 16, __VA_ARGS__);                                    \
            else NC_LAUNCH_PORT(512, 4, kSplitMC, __VA_ARGS__);                                 \
        } else if (c_.ppt == 4) {                                                               \
            if (w_) NC_LAUNCH_PORT(1024, 4, 8, __VA_ARGS__);                                    \
            else NC_LAUNCH_PORT(1024, 4, kSplitMC, __VA_ARGS__);                                \
        } else {                                                                                \
            NC_LAUNCH_PORT(1024, 8, 4, __VA_ARGS__);                                            \
        }                                                                                       \
    } while (0)

}  // namespace

extern "C" {

size_t nc_epilogue_workspace_size(int B, int M, int h, int w) {
    if (B <= 0 || M <= 0 || h <= 0 || w <= 0) return 0;
    return epi_ws(nullptr, B, M, h * w).bytes;
}

int nc_epilogue_fwd_partials(int B, int M, int h, int w) {
    if (B <= 0 || M <= 0 || h <= 0 || w <= 0) return 0;
    return h * w <= kSingleMaxPix ? fwd_plan(B, M, h * w).G : 1;
}

// The tiled forward's second stage from tile statistics (Ts tiles of tn pixels per plane).
static int tile_fwd(hipStream_t st, bool vec, int act, int B, int M, int N, int Ts, int tn,
             float neg_slope, int has_border, const float* z, const float* delta,
             const float* w_eff, const float* s_eff, const float* b_roi, const float* stats,
             float* out, float* mean, float* rstd) {
    const int T = tiles_of(N);
    return dispatch_act(act, [&]<int ACT>() {
        if (vec)
            hipLaunchKernelGGL((k_tile_fwd<ACT, true>), dim3(T, B), dim3(kTileNT), 0, st, B, M,
                               N, Ts, tn, neg_slope, has_border, z, delta, w_eff, s_eff, b_roi,
                               stats, out, mean, rstd);
        else
            hipLaunchKernelGGL((k_tile_fwd<ACT, false>), dim3(T, B), dim3(kTileNT), 0, st, B, M,
                               N, Ts, tn, neg_slope, has_border, z, delta, w_eff, s_eff, b_roi,
                               stats, out, mean, rstd);
        NC_CHECK_LAUNCH();
        return NC_OK;
    });
}

// parts != nullptr: the G direction-group partial outputs go there, uncombined.
static int epilogue_fwd(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                        int has_border, const float* z, const float* delta, const float* w_eff,
                        const float* s_eff, const float* b_roi, float* out, float* parts,
                        float* mean, float* rstd, void* ws, size_t ws_bytes) {
    if (B <= 0 || M <= 0 || M > kMaxM || h <= 0 || w <= 0 || !z || !w_eff || !s_eff ||
        !b_roi || !(out || parts) || !mean || !rstd || (has_border && !delta) || act < 0 ||
        act > 5)
        return NC_ERR_INVALID_ARGUMENT;
    if (ws_bytes < nc_epilogue_workspace_size(B, M, h, w) || !ws) return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
    const int N = h * w;
    const EpiWs e = epi_ws(ws, B, M, N);
    if (parts) out = parts;  // a single group (or the tiled pipeline) writes the output itself
    if (N <= kSingleMaxPix) {
        const DirPlan P = fwd_plan(B, M, N);
        return dispatch_act(act, [&]<int ACT>() {
            NC_FWD_DISPATCH(P, k_epi_fwd, dim3(B, P.G), dim3(P.c.nt), 0, st, M, N, P.mpg,
                            neg_slope, has_border, z, delta, w_eff, s_eff, b_roi, out, mean, rstd,
                            parts ? parts : e.fpart);
            NC_CHECK_LAUNCH();
            if (P.G > 1 && !parts) {
                const size_t n = (size_t)B * N;
                hipLaunchKernelGGL(k_group_sum, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                                   st, P.G, n, e.fpart, out);
                NC_CHECK_LAUNCH();
            }
            return NC_OK;
        });
    }
    const int T = tiles_of(N);
    const bool vec = tile_vec(N, has_border, z, delta, w_eff, s_eff, b_roi);
    tile_stats(st, vec, B, M, N, T, has_border, z, delta, e.stats);
    NC_CHECK_LAUNCH();
    return tile_fwd(st, vec, act, B, M, N, T, kTileN, neg_slope, has_border, z, delta, w_eff,
                    s_eff, b_roi, e.stats, out, mean, rstd);
}

int nc_epilogue_fwd(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                    int has_border, const float* z, const float* delta, const float* w_eff,
                    const float* s_eff, const float* b_roi, float* out, float* mean, float* rstd,
                    void* ws, size_t ws_bytes) {
    if (!out) return NC_ERR_INVALID_ARGUMENT;
    return epilogue_fwd(stream, B, M, h, w, act, neg_slope, has_border, z, delta, w_eff, s_eff,
                        b_roi, out, nullptr, mean, rstd, ws, ws_bytes);
}

int nc_epilogue_fwd_parts(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                          int has_border, const float* z, const float* delta, const float* w_eff,
                          const float* s_eff, const float* b_roi, float* parts, float* mean,
                          float* rstd, void* ws, size_t ws_bytes) {
    if (!parts) return NC_ERR_INVALID_ARGUMENT;
    return epilogue_fwd(stream, B, M, h, w, act, neg_slope, has_border, z, delta, w_eff, s_eff,
                        b_roi, nullptr, parts, mean, rstd, ws, ws_bytes);
}

int nc_epilogue_bwd_partials(int B, int M, int h, int w) {
    if (B <= 0 || M <= 0 || h <= 0 || w <= 0) return 0;
    return h * w <= kSingleMaxPix ? bwd_plan(B, M, h * w).G * B : B;
}

// pg_rows != nullptr: the gw / gs / gb partial rows go there (planes plane_stride floats
// apart) and are not reduced; otherwise to the workspace, reduced into gw / gs / gb.
static int epilogue_bwd(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                        int has_border, const float* z, const float* delta, const float* w_eff,
                        const float* s_eff, const float* b_roi, const float* mean,
                        const float* rstd, const float* gy, float* gz, float* gdb, float* gw,
                        float* gs, float* gb, int accumulate_params, int accumulate_gdb,
                        float* pg_rows, size_t plane_stride, void* ws, size_t ws_bytes) {
    if (B <= 0 || M <= 0 || M > kMaxM || h <= 0 || w <= 0 || !z || !w_eff || !s_eff ||
        !b_roi || !mean || !rstd || !gy || !gz || (!pg_rows && (!gw || !gs || !gb)) ||
        (has_border && !delta) || act < 0 || act > 5)
        return NC_ERR_INVALID_ARGUMENT;
    if (ws_bytes < nc_epilogue_workspace_size(B, M, h, w) || !ws) return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
    const int N = h * w;
    const EpiWs e = epi_ws(ws, B, M, N);
    const int rows = nc_epilogue_bwd_partials(B, M, h, w);  // rows of each pg partial plane
    float* pg = pg_rows ? pg_rows : e.pg;
    const size_t RN = pg_rows ? plane_stride : (size_t)rows * N;
    if (pg_rows && plane_stride < (size_t)rows * N) return NC_ERR_INVALID_ARGUMENT;
    int rc = dispatch_act(act, [&]<int ACT>() {
        if (N <= kSingleMaxPix) {
            const DirPlan P = bwd_plan(B, M, N);
            // the pixel mapping (and so the reduction order) depends only on the operands'
            // alignment: both forms of the entry point give bit-identical results
            const bool vec = N % 4 == 0 && aligned16(z) && aligned16(gz) &&
                             (!has_border || aligned16(delta)) && aligned16(w_eff) &&
                             aligned16(s_eff) && aligned16(b_roi) && aligned16(gy);
            NC_BWD_DISPATCH(P, vec, dim3(B, P.G), dim3(P.c.nt), 0, st, M, N, P.mpg,
                            neg_slope, has_border, z, delta, w_eff, s_eff, b_roi, mean, rstd, gy,
                            gz, pg, RN);
            NC_CHECK_LAUNCH();
            return NC_OK;
        }
        const int T = tiles_of(N);
        const bool tv = tile_vec(N, has_border, z, delta, w_eff, s_eff, b_roi, gy);
#define NC_TILE_BWD(V_)                                                                       \
    do {                                                                                      \
        hipLaunchKernelGGL((k_tile_bwd1<ACT, V_>), dim3(T, B), dim3(kTileNT), 0, st, B, M, N, \
                           T, neg_slope, has_border, z, delta, w_eff, s_eff, b_roi, mean,     \
                           rstd, gy, e.stats, pg, RN);                                        \
        NC_CHECK_LAUNCH();                                                                    \
        hipLaunchKernelGGL((k_tile_bwd2<ACT, V_>), dim3(T, M, B), dim3(kTileNT), 0, st, B, M, \
                           N, T, neg_slope, has_border, z, delta, w_eff, s_eff, b_roi, mean,  \
                           rstd, gy, e.stats, gz);                                            \
        NC_CHECK_LAUNCH();                                                                    \
    } while (0)
        if (tv) NC_TILE_BWD(true);
        else NC_TILE_BWD(false);
#undef NC_TILE_BWD
        return NC_OK;
    });
    if (rc != NC_OK) return rc;
    // parameter gradients and the border cotangent: sums over the partial rows (gw, gs, gb
    // planes of pg) and over B of gz, in one launch
    const bool own = pg_rows == nullptr;
    const RedJob jobs[4] = {{own ? pg : nullptr, gw, N, accumulate_params, rows},
                            {own ? pg + RN : nullptr, gs, N, accumulate_params, rows},
                            {own ? pg + 2 * RN : nullptr, gb, N, accumulate_params, rows},
                            {has_border ? gz : nullptr, gdb, M * N, accumulate_gdb,
                             has_border ? B : 0}};  // without the border term gdb = 0
    return launch_batch_reduce(st, jobs, 4);
}

int nc_epilogue_bwd(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                    int has_border, const float* z, const float* delta, const float* w_eff,
                    const float* s_eff, const float* b_roi, const float* mean, const float* rstd,
                    const float* gy, float* gz, float* gdb, float* gw, float* gs, float* gb,
                    int accumulate_params, int accumulate_gdb, void* ws, size_t ws_bytes) {
    return epilogue_bwd(stream, B, M, h, w, act, neg_slope, has_border, z, delta, w_eff, s_eff,
                        b_roi, mean, rstd, gy, gz, gdb, gw, gs, gb, accumulate_params,
                        accumulate_gdb, nullptr, 0, ws, ws_bytes);
}

// ----------------------------------------------------------------------------------------
// Plain per-plane standardisation (epilogue.py:20-25 standardize_spatial_nchw) and its
// reverse: one 256-thread workgroup per (b, m) plane, two-pass population statistics with
// eps = 1e-5 inside the square root, as every epilogue kernel here; the reverse recomputes
// zhat from the saved (mean, rstd).
// ----------------------------------------------------------------------------------------

namespace {

constexpr int kStdNT = 256;

__global__ __launch_bounds__(kStdNT) void k_std_fwd(int n, const float* __restrict__ x,
                                                    float* __restrict__ out,
                                                    float* __restrict__ mean,
                                                    float* __restrict__ rstd) {
    __shared__ float red[2 * (kStdNT / NC_WAVE) + 2];
    const size_t base = (size_t)blockIdx.x * n;
    const float* xp = x + base;
    float v[1] = {0.0f};
    for (int i = threadIdx.x; i < n; i += kStdNT) v[0] += xp[i];
    block_sum<1, kStdNT>(v, red);
    const float inv_n = 1.0f / (float)n;
    const float mu = v[0] * inv_n;
    v[0] = 0.0f;
    for (int i = threadIdx.x; i < n; i += kStdNT) {
        const float d = xp[i] - mu;
        v[0] = fmaf(d, d, v[0]);
    }
    block_sum<1, kStdNT>(v, red);
    const float r = 1.0f / sqrtf(v[0] * inv_n + 1e-5f);
    for (int i = threadIdx.x; i < n; i += kStdNT) out[base + i] = (xp[i] - mu) * r;
    if (threadIdx.x == 0) {
        mean[blockIdx.x] = mu;
        rstd[blockIdx.x] = r;
    }
}

// gx = rstd * (g - mean(g) - zhat * mean(g * zhat)), zhat = (x - mean) * rstd.
__global__ __launch_bounds__(kStdNT) void k_std_bwd(int n, const float* __restrict__ x,
                                                    const float* __restrict__ mean,
                                                    const float* __restrict__ rstd,
                                                    const float* __restrict__ g,
                                                    float* __restrict__ gx) {
    __shared__ float red[2 * (kStdNT / NC_WAVE) + 4];
    const size_t base = (size_t)blockIdx.x * n;
    const float mu = mean[blockIdx.x], r = rstd[blockIdx.x];
    float v[2] = {0.0f, 0.0f};
    for (int i = threadIdx.x; i < n; i += kStdNT) {
        const float gi = g[base + i];
        v[0] += gi;
        v[1] = fmaf(gi, (x[base + i] - mu) * r, v[1]);
    }
    block_sum<2, kStdNT>(v, red);
    const float inv_n = 1.0f / (float)n;
    const float c1 = v[0] * inv_n, c2 = v[1] * inv_n;
    for (int i = threadIdx.x; i < n; i += kStdNT) {
        const float zh = (x[base + i] - mu) * r;
        gx[base + i] = r * (g[base + i] - c1 - zh * c2);
    }
}

}  // namespace

int nc_standardize_fwd(void* stream, int nplanes, int n, const float* x, float* out,
                       float* mean, float* rstd) {
    if (nplanes <= 0 || n <= 0 || !x || !out || !mean || !rstd) return NC_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_std_fwd, dim3(nplanes), dim3(kStdNT), 0, nc_stream(stream), n, x, out,
                       mean, rstd);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_standardize_bwd(void* stream, int nplanes, int n, const float* x, const float* mean,
                       const float* rstd, const float* g, float* gx) {
    if (nplanes <= 0 || n <= 0 || !x || !mean || !rstd || !g || !gx)
        return NC_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_std_bwd, dim3(nplanes), dim3(kStdNT), 0, nc_stream(stream), n, x, mean,
                       rstd, g, gx);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

// ----------------------------------------------------------------------------------------
// Allocation-free variant of nc_epilogue_bwd: its scratch (the per-(group, sample) partial
// rows and the tile statistics, nc_epilogue_workspace_size bytes) lives in file-scope device
// memory instead of a caller workspace.  Each GPU holds its own copy of the array from the
// library's load until the process ends.  The host-side name `scratch` is only a stand-in
// symbol: its device address is looked up once per device (hipGetSymbolAddress, that device
// current) and that address is what the kernels receive.  Every call on a GPU shares the
// GPU's array: calls that overlap on one GPU race.  No kernel here needs the scratch zeroed:
// every partial row and tile statistic is written before it is read.
// ----------------------------------------------------------------------------------------

static __device__ __align__(256) unsigned char scratch[NC_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxScratchDevices] = {};

// The current device's address of `scratch`, looked up on its first use on that device.
int scratch_address(void** addr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxScratchDevices) return NC_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return NC_ERR_WORKSPACE;
        g_scratch_addr[dev] = p;
    }
    *addr = g_scratch_addr[dev];
    return NC_OK;
}

}  // namespace

int nc_epilogue_bwd_noalloc(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                            int has_border, const float* z, const float* delta,
                            const float* w_eff, const float* s_eff, const float* b_roi,
                            const float* mean, const float* rstd, const float* gy, float* gz,
                            float* gdb, float* gw, float* gs, float* gb, int accumulate_params,
                            int accumulate_gdb) {
    if (B <= 0 || M <= 0 || h <= 0 || w <= 0) return NC_ERR_INVALID_ARGUMENT;
    const size_t need = nc_epilogue_workspace_size(B, M, h, w);
    if (need > sizeof(scratch)) return NC_ERR_SCRATCH_LIMIT;
    if (stream) {  // the stream must belong to the current device, whose scratch is used
        int sdev = -1, cur = -1;
        hipError_t e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
        if (e != hipSuccess) return (int)e;
        e = hipGetDevice(&cur);
        if (e != hipSuccess) return (int)e;
        if (sdev != cur) return NC_ERR_INVALID_ARGUMENT;
    }
    void* ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc != NC_OK) return rc;
    return epilogue_bwd(stream, B, M, h, w, act, neg_slope, has_border, z, delta, w_eff, s_eff,
                        b_roi, mean, rstd, gy, gz, gdb, gw, gs, gb, accumulate_params,
                        accumulate_gdb, nullptr, 0, ws, sizeof(scratch));
}

int nc_epilogue_bwd_parts(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                          int has_border, const float* z, const float* delta, const float* w_eff,
                          const float* s_eff, const float* b_roi, const float* mean,
                          const float* rstd, const float* gy, float* gz, float* pg_rows,
                          size_t plane_stride, void* ws, size_t ws_bytes) {
    if (!pg_rows) return NC_ERR_INVALID_ARGUMENT;
    return epilogue_bwd(stream, B, M, h, w, act, neg_slope, has_border, z, delta, w_eff, s_eff,
                        b_roi, mean, rstd, gy, gz, nullptr, nullptr, nullptr, nullptr, 0, 0,
                        pg_rows, plane_stride, ws, ws_bytes);
}

namespace {

// The dense port's finish: out = fact(sum of the G direction-group partials), fixed order.
__global__ __launch_bounds__(256) void k_port_dense_fwd(int n, int G, int fact, float slope,
                                                        const float* __restrict__ parts,
                                                        float* __restrict__ out,
                                                        float* __restrict__ pre) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float y = parts[i];
    for (int g = 1; g < G; ++g) y += parts[(size_t)g * n + i];
    if (pre) pre[i] = y;
    out[i] = fact == NC_ACT_IDENTITY ? y : nc_act(y, fact, slope);
}

__global__ __launch_bounds__(256) void k_port_dense_bwd(int n, int fact, float slope,
                                                        const float* __restrict__ pre,
                                                        const float* __restrict__ g_out,
                                                        float* __restrict__ g_pre) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float a;
    g_pre[i] = g_out[i] * nc_act_d(pre[i], fact, slope, &a);
}

}  // namespace

int nc_port_dense_fwd(void* stream, int n, int G, int final_act, float neg_slope,
                      const float* parts, float* out, float* pre) {
    if (n <= 0 || G <= 0 || !parts || !out || final_act < 0 || final_act > 5 ||
        (final_act != NC_ACT_IDENTITY && !pre))
        return NC_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_port_dense_fwd, dim3((n + 255) / 256), dim3(256), 0,
                       nc_stream(stream), n, G, final_act, neg_slope, parts, out, pre);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_port_dense_bwd(void* stream, int n, int final_act, float neg_slope, const float* pre,
                      const float* g_out, float* g_pre) {
    if (n <= 0 || !pre || !g_out || !g_pre || final_act <= NC_ACT_IDENTITY || final_act > 5)
        return NC_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_port_dense_bwd, dim3((n + 255) / 256), dim3(256), 0,
                       nc_stream(stream), n, final_act, neg_slope, pre, g_out, g_pre);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_rows_sum(void* stream, int n_jobs, const nc_rows_job* jobs) {
    if (n_jobs <= 0 || n_jobs > kRedJobs || !jobs) return NC_ERR_INVALID_ARGUMENT;
    RedJob rj[kRedJobs];
    for (int i = 0; i < n_jobs; ++i) {
        const nc_rows_job& j = jobs[i];
        if (!j.rows || !j.out || j.nrows <= 0 || j.len <= 0) return NC_ERR_INVALID_ARGUMENT;
        rj[i] = RedJob{j.rows, j.out, j.len, j.accumulate, j.nrows, 1};
    }
    return launch_batch_reduce(nc_stream(stream), rj, n_jobs);
}

static int port_check(int B, int M, int h, int w, int P, const int32_t* port_idx,
                      const float* z, int hb, const float* delta, int fact) {
    if (B <= 0 || M <= 0 || M > kMaxM || h <= 0 || w <= 0 || P <= 0 || P > 256 ||
        M * P > 8192 || !port_idx || !z || (hb && !delta) || fact < 0 || fact > 5)
        return NC_ERR_INVALID_ARGUMENT;
    return NC_OK;
}

int nc_port_fwd(void* stream, int B, int M, int h, int w, int has_border, int final_act,
                float neg_slope, int n_port, const int32_t* port_idx, const float* z,
                const float* delta, const float* port_params, float* out, float* zo,
                float* mean, float* rstd, float* pre, void* ws, size_t ws_bytes) {
    int rc = port_check(B, M, h, w, n_port, port_idx, z, has_border, delta, final_act);
    if (rc != NC_OK) return rc;
    if (!zo || !mean || !rstd || (port_params && !out) ||
        (port_params && final_act != NC_ACT_IDENTITY && !pre))
        return NC_ERR_INVALID_ARGUMENT;
    if (ws_bytes < nc_epilogue_workspace_size(B, M, h, w) || !ws) return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
    const int N = h * w;
    const EpiWs e = epi_ws(ws, B, M, N);
    if (N <= kSingleMaxPix) {
        const DirPlan P = fwd_plan(B, M, N);
        const size_t shm = (size_t)P.mpg * n_port * sizeof(float);
        NC_PORT_DISPATCH(P, dim3(B, P.G), dim3(P.c.nt), shm, st, M, N, P.mpg, n_port,
                         has_border, final_act, neg_slope, port_idx, z, delta, port_params, out,
                         zo, mean, rstd, pre, e.portpart);
        NC_CHECK_LAUNCH();
        if (P.G > 1 && port_params) {
            hipLaunchKernelGGL(k_port_combine, dim3((B * n_port + 255) / 256), dim3(256), 0, st, B,
                               M, n_port, P.G, final_act, neg_slope, port_params, e.portpart, out,
                               pre);
            NC_CHECK_LAUNCH();
        }
        return NC_OK;
    }
    const int T = tiles_of(N);
    tile_stats(st, N % 4 == 0 && aligned16(z) && (!has_border || aligned16(delta)), B, M, N, T,
               has_border, z, delta, e.stats);
    NC_CHECK_LAUNCH();
    const size_t shm = (size_t)M * n_port * sizeof(float);
    hipLaunchKernelGGL(k_port_fwd_tiled, dim3(B), dim3(256), shm, st, B, M, N, T, n_port,
                       has_border, final_act, neg_slope, port_idx, z, delta, port_params,
                       e.stats, out, zo, mean, rstd, pre);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

static int port_bwd(void* stream, int B, int M, int h, int w, int has_border, int final_act,
                    float neg_slope, int n_port, const int32_t* port_idx, const float* z,
                    const float* delta, const float* port_params, const float* zo,
                    const float* mean, const float* rstd, const float* pre, const float* g_out,
                    float* gz, float* gdb, float* g_port_params, int accumulate_params,
                    float* pp_rows, size_t plane_stride, void* ws, size_t ws_bytes) {
    int rc = port_check(B, M, h, w, n_port, port_idx, z, has_border, delta, final_act);
    if (rc != NC_OK) return rc;
    if (!zo || !mean || !rstd || !g_out || !gz ||
        (port_params && !g_port_params && !pp_rows) ||
        (port_params && final_act != NC_ACT_IDENTITY && !pre))
        return NC_ERR_INVALID_ARGUMENT;
    if (pp_rows && plane_stride < (size_t)B * n_port) return NC_ERR_INVALID_ARGUMENT;
    if (ws_bytes < nc_epilogue_workspace_size(B, M, h, w) || !ws) return NC_ERR_WORKSPACE;
    hipStream_t st = nc_stream(stream);
    const int N = h * w;
    const int T = (N + kPortTile - 1) / kPortTile;
    const EpiWs e = epi_ws(ws, B, M, N);
    float* ppart = pp_rows ? pp_rows : e.pport;
    const size_t ps = pp_rows ? plane_stride : (size_t)B * n_port;
    const size_t shm = (size_t)3 * M * n_port * sizeof(float) + (size_t)kPortTile * sizeof(int);
    const dim3 grid(T, (M + kPortMC - 1) / kPortMC, B);
    if (N % 4 == 0 && aligned16(z) && aligned16(gz) && (!has_border || aligned16(delta)))
        hipLaunchKernelGGL(k_port_bwd<true>, grid, dim3(kPortNT), shm, st, M, N, n_port,
                           has_border, final_act, neg_slope, port_idx, z, delta, port_params, zo,
                           mean, rstd, pre, g_out, gz, ppart, ps);
    else
        hipLaunchKernelGGL(k_port_bwd<false>, grid, dim3(kPortNT), shm, st, M, N, n_port,
                           has_border, final_act, neg_slope, port_idx, z, delta, port_params, zo,
                           mean, rstd, pre, g_out, gz, ppart, ps);
    NC_CHECK_LAUNCH();
    // port-parameter gradients (3 rows of P) and the border cotangent, in one launch
    const bool pj = port_params != nullptr && pp_rows == nullptr;
    const RedJob jobs[4] = {
        {pj ? ppart : nullptr, g_port_params, n_port, accumulate_params, B},
        {pj ? ppart + ps : nullptr, g_port_params + n_port, n_port, accumulate_params, B},
        {pj ? ppart + 2 * ps : nullptr, g_port_params + 2 * n_port, n_port, accumulate_params,
         B},
        {has_border ? gz : nullptr, gdb, M * N, accumulate_params, has_border ? B : 0}};
    return launch_batch_reduce(st, jobs, 4);
}

int nc_port_bwd(void* stream, int B, int M, int h, int w, int has_border, int final_act,
                float neg_slope, int n_port, const int32_t* port_idx, const float* z,
                const float* delta, const float* port_params, const float* zo,
                const float* mean, const float* rstd, const float* pre, const float* g_out,
                float* gz, float* gdb, float* g_port_params, int accumulate_params, void* ws,
                size_t ws_bytes) {
    return port_bwd(stream, B, M, h, w, has_border, final_act, neg_slope, n_port, port_idx, z,
                    delta, port_params, zo, mean, rstd, pre, g_out, gz, gdb, g_port_params,
                    accumulate_params, nullptr, 0, ws, ws_bytes);
}

int nc_port_bwd_parts(void* stream, int B, int M, int h, int w, int has_border, int final_act,
                      float neg_slope, int n_port, const int32_t* port_idx, const float* z,
                      const float* delta, const float* port_params, const float* zo,
                      const float* mean, const float* rstd, const float* pre,
                      const float* g_out, float* gz, float* pp_rows, size_t plane_stride,
                      void* ws, size_t ws_bytes) {
    if (!pp_rows || !port_params) return NC_ERR_INVALID_ARGUMENT;
    return port_bwd(stream, B, M, h, w, has_border, final_act, neg_slope, n_port, port_idx, z,
                    delta, port_params, zo, mean, rstd, pre, g_out, gz, nullptr, nullptr, 0,
                    pp_rows, plane_stride, ws, ws_bytes);
}

}  // extern "C"

bool nc_epilogue_tiled(int n_pix) { return n_pix > kSingleMaxPix; }

int nc_epilogue_bwd_stage1(hipStream_t st, int B, int M, int h, int w, int act, float neg_slope,
                           const float* z, const float* w_eff, const float* s_eff,
                           const float* b_roi, const float* mean, const float* rstd,
                           const float* gy, float* pg_rows, size_t plane_stride, void* ws,
                           size_t ws_bytes, const float** cpart, int* n_tiles) {
    const int N = h * w;
    if (B <= 0 || M <= 0 || M > kMaxM || h <= 0 || w <= 0 || !nc_epilogue_tiled(N) || !z ||
        !w_eff || !s_eff || !b_roi || !mean || !rstd || !gy || !pg_rows || act < 0 || act > 5 ||
        plane_stride < (size_t)B * N || !cpart || !n_tiles)
        return NC_ERR_INVALID_ARGUMENT;
    if (ws_bytes < nc_epilogue_workspace_size(B, M, h, w) || !ws) return NC_ERR_WORKSPACE;
    const EpiWs e = epi_ws(ws, B, M, N);
    const int T = tiles_of(N);
    // the same pixel mapping (and so the same c1 / c2 partials) as nc_epilogue_bwd_parts
    const bool tv = tile_vec(N, 0, z, nullptr, w_eff, s_eff, b_roi, gy);
    int rc = dispatch_act(act, [&]<int ACT>() {
        if (tv)
            hipLaunchKernelGGL((k_tile_bwd1<ACT, true>), dim3(T, B), dim3(kTileNT), 0, st, B, M,
                               N, T, neg_slope, 0, z, nullptr, w_eff, s_eff, b_roi, mean, rstd,
                               gy, e.stats, pg_rows, plane_stride);
        else
            hipLaunchKernelGGL((k_tile_bwd1<ACT, false>), dim3(T, B), dim3(kTileNT), 0, st, B,
                               M, N, T, neg_slope, 0, z, nullptr, w_eff, s_eff, b_roi, mean,
                               rstd, gy, e.stats, pg_rows, plane_stride);
        NC_CHECK_LAUNCH();
        return NC_OK;
    });
    *cpart = e.stats;
    *n_tiles = T;
    return rc;
}

int nc_epilogue_fwd_from_stats(hipStream_t st, int B, int M, int h, int w, int act,
                               float neg_slope, const float* z, const float* w_eff,
                               const float* s_eff, const float* b_roi, const float* stats,
                               int n_tiles, int tile_pix, float* out, float* mean, float* rstd) {
    const int N = h * w;
    if (B <= 0 || M <= 0 || M > kMaxM || !nc_epilogue_tiled(N) || !z || !w_eff || !s_eff ||
        !b_roi || !stats || !out || !mean || !rstd || act < 0 || act > 5 || tile_pix <= 0 ||
        n_tiles != (N + tile_pix - 1) / tile_pix)
        return NC_ERR_INVALID_ARGUMENT;
    return tile_fwd(st, tile_vec(N, 0, z, nullptr, w_eff, s_eff, b_roi), act, B, M, N, n_tiles,
                    tile_pix, neg_slope, 0, z, nullptr, w_eff, s_eff, b_roi, stats, out, mean,
                    rstd);
}

// The port algebra over G direction-group partial sums part (2, G, B, P), for producers in
// other translation units (the fused correlation + port of the spectral entry points).
int nc_port_combine_launch(hipStream_t st, int B, int M, int P, int G, int final_act,
                           float neg_slope, const float* port_params, const float* part,
                           float* out, float* pre) {
    hipLaunchKernelGGL(k_port_combine, dim3((B * P + 255) / 256), dim3(256), 0, st, B, M, P, G,
                       final_act, neg_slope, port_params, part, out, pre);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

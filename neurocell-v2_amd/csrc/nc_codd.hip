// Piece 1 (pre-step Codd fusion), piece 4 (adaptive active-region statistics) and the small
// orchestration kernels (input injection, MSE loss, AdamW).
//
// The pre-step fusion is latency-bound (one (3,H,W) pass per batch): one thread per grid
// cell evaluates the pinned weight, the Codd probability in the requested mode and the
// border template, and scatters each into the (possibly cropped) ROI operands; the port
// parameters are gathered by P extra threads.  The backward is the same map transposed.
#include <math.h>

#include "nc_common.h"

namespace {

struct CellEval {
    float w_pinned, s_prob, ds, b;
};

// params.py:31-80 (compute_codd_state_probs) and params.py:249 (output-weight pin).
NC_DEV CellEval eval_cell(const nc_chip_desc& c, const float* cell, const uint8_t* io,
                          const uint8_t* owm, int mode, float inv_tau, float thr, int hard_pin,
                          int idx) {
    const size_t HW = (size_t)c.H * c.W;
    const float w = cell[idx], b = cell[HW + idx], s = cell[2 * HW + idx];
    const bool pin = io[idx] != 0;
    CellEval e;
    e.b = b;
    e.w_pinned = owm[idx] ? 1.0f : w;
    const float base = (!hard_pin && pin) ? 1.0f : s;
    float p, d;
    if (mode == NC_CODD_CONTINUOUS) {
        p = nc_sigmoid(base);
        d = p * (1.0f - p);
    } else {
        const float soft = nc_sigmoid(base * inv_tau);
        d = inv_tau * soft * (1.0f - soft);
        if (mode == NC_CODD_ANNEALED) {
            p = soft;
        } else {
            float hard;
            if (mode == NC_CODD_STE_BINARY)
                hard = base >= 0.0f ? 1.0f : 0.0f;
            else
                hard = base >= thr ? 1.0f : (base > 0.0f ? 0.5f : 0.0f);
            p = soft + (hard - soft);  // straight-through: value of hard, gradient of soft
        }
    }
    if (hard_pin && pin) p = 1.0f;
    e.s_prob = p;
    e.ds = pin ? 0.0f : d;  // constant (pinned) at I/O cells in both pin variants
    return e;
}

NC_DEV bool in_roi(const nc_chip_desc& c, int r, int col) {
    return r >= c.pad_h && r < c.H - c.pad_h && col >= c.pad_w && col < c.W - c.pad_w;
}

NC_DEV void codd_fwd_at(int q, const nc_chip_desc& c, const float* __restrict__ cell,
                        const uint8_t* __restrict__ io, const uint8_t* __restrict__ owm,
                        int mode, float inv_tau, float thr, int hard_pin, int act, float slope,
                        int P, const int* __restrict__ prc, float* __restrict__ w_eff,
                        float* __restrict__ s_eff, float* __restrict__ b_roi,
                        float* __restrict__ patch, float* __restrict__ pp,
                        float* __restrict__ s_prob, float* __restrict__ border2d,
                        float* __restrict__ w_pin) {
    const int HW = c.H * c.W;
    const float inv_m = 1.0f / (float)c.M;
    if (q < HW) {
        const int r = q / c.W, col = q % c.W;
        CellEval e = eval_cell(c, cell, io, owm, mode, inv_tau, thr, hard_pin, q);
        if (s_prob) s_prob[q] = e.s_prob;
        if (w_pin) w_pin[q] = e.w_pinned;
        if (border2d) border2d[q] = nc_act(e.b, act, slope) * e.s_prob;
        const int h = c.r1 - c.r0, w = c.c1 - c.c0;
        const int ri = r - c.pad_h - c.r0, ci = col - c.pad_w - c.c0;
        if (ri >= 0 && ri < h && ci >= 0 && ci < w) {  // active sub-ROI (params.py:259-275)
            const int o = ri * w + ci;
            w_eff[o] = inv_m * e.w_pinned * (1.0f - e.s_prob);
            s_eff[o] = inv_m * e.s_prob;
            b_roi[o] = e.b;
        }
        // border template, ROI zeroed, cut to the sub-ROI's receptive field
        // (params.py:277-279, propagator.py:355-361)
        const int Hp = h + c.kh - 1, Wp = w + c.kw - 1;
        const int pi = r - c.r0, pj = col - c.c0;
        if (pi >= 0 && pi < Hp && pj >= 0 && pj < Wp)
            patch[pi * Wp + pj] = in_roi(c, r, col) ? 0.0f : nc_act(e.b, act, slope) * e.s_prob;
    } else if (q < HW + P) {
        const int k = q - HW;  // output port cell (params.py:296-301 / :283-289)
        const int r = c.pad_h + prc[k], col = c.pad_w + prc[P + k];
        CellEval e = eval_cell(c, cell, io, owm, mode, inv_tau, thr, hard_pin, r * c.W + col);
        pp[k] = inv_m * e.w_pinned * (1.0f - e.s_prob);
        pp[P + k] = inv_m * e.s_prob;
        pp[2 * P + k] = e.b;
    }
}

__global__ void k_codd_fwd(nc_chip_desc c, const float* __restrict__ cell,
                           const uint8_t* __restrict__ io, const uint8_t* __restrict__ owm,
                           int mode, float inv_tau, float thr, int hard_pin, int act, float slope,
                           int P, const int* __restrict__ prc, float* __restrict__ w_eff,
                           float* __restrict__ s_eff, float* __restrict__ b_roi,
                           float* __restrict__ patch, float* __restrict__ pp,
                           float* __restrict__ s_prob, float* __restrict__ border2d,
                           float* __restrict__ w_pin) {
    codd_fwd_at(blockIdx.x * blockDim.x + threadIdx.x, c, cell, io, owm, mode, inv_tau, thr,
                hard_pin, act, slope, P, prc, w_eff, s_eff, b_roi, patch, pp, s_prob, border2d,
                w_pin);
}

struct InjectArgs {
    int B, n_in, n_roi;
    const float* in;
    const int* src;
    float* roi;
};

// The step's prologue in one launch: the Codd fusion's H*W + P threads, then one thread per
// injected cell (k_inject's map), the two being independent.
__global__ void k_prologue(nc_chip_desc c, const float* __restrict__ cell,
                           const uint8_t* __restrict__ io, const uint8_t* __restrict__ owm,
                           int mode, float inv_tau, float thr, int hard_pin, int act, float slope,
                           int P, const int* __restrict__ prc, float* __restrict__ w_eff,
                           float* __restrict__ s_eff, float* __restrict__ b_roi,
                           float* __restrict__ patch, float* __restrict__ pp,
                           float* __restrict__ s_prob, InjectArgs ia) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t nc = (size_t)c.H * c.W + P;
    if (q < nc) {
        codd_fwd_at((int)q, c, cell, io, owm, mode, inv_tau, thr, hard_pin, act, slope, P, prc,
                    w_eff, s_eff, b_roi, patch, pp, s_prob, nullptr, nullptr);
    } else if (q - nc < (size_t)ia.B * ia.n_roi) {
        const size_t k = q - nc;
        const int b = (int)(k / ia.n_roi), i = (int)(k % ia.n_roi);
        const int e = ia.src[i];
        ia.roi[k] = e >= 0 ? ia.in[(size_t)b * ia.n_in + e] : 0.0f;
    }
}

__global__ void k_codd_bwd(nc_chip_desc c, const float* __restrict__ cell,
                           const uint8_t* __restrict__ io, const uint8_t* __restrict__ owm,
                           int mode, float inv_tau, float thr, int hard_pin, int act, float slope,
                           int P, const int* __restrict__ prc,
                           const int* __restrict__ pc_start, const int* __restrict__ pc_list,
                           const float* __restrict__ g_weff,
                           const float* __restrict__ g_seff, const float* __restrict__ g_broi,
                           const float* __restrict__ g_patch, const float* __restrict__ g_pp,
                           const float* __restrict__ g_sprob, const float* __restrict__ g_bfull,
                           float* __restrict__ g_cell) {
    const int HW = c.H * c.W;
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= HW) return;
    const float inv_m = 1.0f / (float)c.M;
    const int r = q / c.W, col = q % c.W;
    CellEval e = eval_cell(c, cell, io, owm, mode, inv_tau, thr, hard_pin, q);
    float gw = 0.f, gs = 0.f, gb = 0.f, gbd = 0.f;
    const int h = c.r1 - c.r0, w = c.c1 - c.c0;
    const int ri = r - c.pad_h - c.r0, ci = col - c.pad_w - c.c0;
    if (ri >= 0 && ri < h && ci >= 0 && ci < w) {
        const int o = ri * w + ci;
        if (g_weff) gw += g_weff[o];
        if (g_seff) gs += g_seff[o];
        if (g_broi) gb += g_broi[o];
    }
    if (g_pp && in_roi(c, r, col)) {
        const int rr = r - c.pad_h, cc = col - c.pad_w;
        if (pc_start) {  // this cell's ports, in increasing port order
            const int o = rr * c.roi_w + cc;
            for (int i = pc_start[o]; i < pc_start[o + 1]; ++i) {
                const int k = pc_list[i];
                gw += g_pp[k];
                gs += g_pp[P + k];
                gb += g_pp[2 * P + k];
            }
        } else {
            for (int k = 0; k < P; ++k)  // fixed order; duplicates of a port cell add up
                if (prc[k] == rr && prc[P + k] == cc) {
                    gw += g_pp[k];
                    gs += g_pp[P + k];
                    gb += g_pp[2 * P + k];
                }
        }
    }
    const int Hp = h + c.kh - 1, Wp = w + c.kw - 1;
    const int pi = r - c.r0, pj = col - c.c0;
    if (g_patch && pi >= 0 && pi < Hp && pj >= 0 && pj < Wp && !in_roi(c, r, col))
        gbd = g_patch[pi * Wp + pj];
    float a;
    const float da = nc_act_d(e.b, act, slope, &a);
    const float g_wp = inv_m * (1.0f - e.s_prob) * gw;
    const float g_sp = -inv_m * e.w_pinned * gw + inv_m * gs + a * gbd +
                       (g_sprob ? g_sprob[q] : 0.0f);
    const float g_b = gb + da * e.s_prob * gbd + (g_bfull ? g_bfull[q] : 0.0f);
    g_cell[q] = owm[q] ? 0.0f : g_wp;
    g_cell[HW + q] = g_b;
    g_cell[2 * HW + q] = g_sp * e.ds;
}

// ----------------------------------------------------------------------------------------
// Piece 4: _compute_adaptive_mask_tensors (adaptive_mask.py:200-315), one workgroup.
// ----------------------------------------------------------------------------------------

constexpr int kAdNT = 1024;

__global__ __launch_bounds__(kAdNT) void k_adaptive(
    nc_chip_desc c, const float* __restrict__ cell, const float* __restrict__ filt,
    const uint8_t* __restrict__ io_roi, const float* __restrict__ act_roi, int mh, int mw,
    float sal_thr, float bias_thr, float filt_thr, float act_thr, int* __restrict__ stats,
    uint8_t* __restrict__ dil) {
    HIP_DYNAMIC_SHARED(uint8_t, smask)  // 2 * roi_h * roi_w: seed, row-dilated
    __shared__ float red[6 * (kAdNT / 64)];
    __shared__ float peak_s[kAdNT / 64 + 1];
    const int tid = threadIdx.x;
    const int K = c.kh * c.kw, HW = c.H * c.W;
    const int hv = c.roi_h, wv = c.roi_w, N = hv * wv;
    // 1. effective filter radii
    float pk = 0.f;
    for (int t = tid; t < K; t += kAdNT) {
        float mx = 0.f;
        for (int m = 0; m < c.M; ++m) mx = fmaxf(mx, fabsf(filt[(size_t)m * K + t]));
        pk = fmaxf(pk, mx);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) pk = fmaxf(pk, __shfl_xor(pk, off, NC_WAVE));
    if ((tid & 63) == 0) peak_s[tid >> 6] = pk;
    __syncthreads();
    float peak = 0.f;
    for (int wv_ = 0; wv_ < kAdNT / 64; ++wv_) peak = fmaxf(peak, peak_s[wv_]);
    const float tap_thr = filt_thr * peak + 1e-12f;
    float rh = 0.f, rw = 0.f;
    for (int t = tid; t < K; t += kAdNT) {
        float mx = 0.f;
        for (int m = 0; m < c.M; ++m) mx = fmaxf(mx, fabsf(filt[(size_t)m * K + t]));
        if (mx >= tap_thr) {
            rh = fmaxf(rh, fabsf((float)(t / c.kw - (c.kh - 1) / 2)));
            rw = fmaxf(rw, fabsf((float)(t % c.kw - (c.kw - 1) / 2)));
        }
    }
    // 2. salience moments (fixed-order sums)
    float v[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // upd_cnt, drive_sum, nonio_cnt, wmag_sum
    for (int i = tid; i < N; i += kAdNT) {
        const int g = (c.pad_h + i / wv) * c.W + c.pad_w + i % wv;
        const float b = cell[HW + g], sp = nc_sigmoid(cell[2 * HW + g]), w = cell[g];
        const bool nonio = io_roi[i] == 0;
        const bool upd = nonio && fabsf(b) > 1e-5f;
        if (upd) {
            v[0] += 1.f;
            v[1] += fabsf(b) * sp;
        }
        if (nonio) {
            v[2] += 1.f;
            v[3] += fabsf(w) * sp;
        }
    }
    block_sum<4, kAdNT>(v, red);
    const float upd_cnt = fmaxf(1.f, v[0]), nonio_cnt = fmaxf(1.f, v[2]);
    const float b_mean = v[1] / upd_cnt, w_mean = v[3] / nonio_cnt;
    float q2[2] = {0.f, 0.f};
    for (int i = tid; i < N; i += kAdNT) {
        const int g = (c.pad_h + i / wv) * c.W + c.pad_w + i % wv;
        const float b = cell[HW + g], sp = nc_sigmoid(cell[2 * HW + g]), w = cell[g];
        const bool nonio = io_roi[i] == 0;
        if (nonio && fabsf(b) > 1e-5f) {
            const float d = fabsf(b) * sp - b_mean;
            q2[0] += d * d;
        }
        if (nonio) {
            const float d = fabsf(w) * sp - w_mean;
            q2[1] += d * d;
        }
    }
    block_sum<2, kAdNT>(q2, red);
    const float b_std = sqrtf(q2[0] / upd_cnt), w_std = sqrtf(q2[1] / nonio_cnt);
    // 3. seed mask
    float cnt = 0.f;
    for (int i = tid; i < N; i += kAdNT) {
        const int g = (c.pad_h + i / wv) * c.W + c.pad_w + i % wv;
        const float b = cell[HW + g], sp = nc_sigmoid(cell[2 * HW + g]), w = cell[g];
        const bool nonio = io_roi[i] == 0;
        const float drive = fabsf(b) * sp;
        const float zb = (drive - b_mean) / (b_std + 1e-6f);
        const bool sal_b = nonio && sp > 0.5f && drive > bias_thr &&
                           (zb > sal_thr || drive > 4.0f * bias_thr);
        const float zw = (fabsf(w) * sp - w_mean) / (w_std + 1e-6f);
        const bool sal_r = nonio && fabsf(b) > 0.5f * bias_thr && zw > sal_thr && sp > 0.85f;
        bool seed = !nonio || sal_b || sal_r;
        if (act_roi) seed = seed || act_roi[i] > act_thr;
        smask[i] = seed ? 1 : 0;
        cnt += seed ? 1.f : 0.f;
    }
    __syncthreads();
    // 4. separable rectangular dilation ("SAME" max-pool): rows then columns
    uint8_t* rowd = smask + N;
    for (int i = tid; i < N; i += kAdNT) {
        const int r = i / wv, col = i % wv;
        uint8_t any = 0;
        for (int d = max(0, col - mw); d <= min(wv - 1, col + mw); ++d) any |= smask[r * wv + d];
        rowd[i] = any;
    }
    __syncthreads();
    float bb[4] = {(float)hv, -1.f, (float)wv, -1.f};  // rmin, rmax, cmin, cmax
    for (int i = tid; i < N; i += kAdNT) {
        const int r = i / wv, col = i % wv;
        uint8_t any = 0;
        for (int d = max(0, r - mh); d <= min(hv - 1, r + mh); ++d) any |= rowd[d * wv + col];
        dil[i] = any;
        if (any) {
            bb[0] = fminf(bb[0], (float)r);
            bb[1] = fmaxf(bb[1], (float)r);
            bb[2] = fminf(bb[2], (float)col);
            bb[3] = fmaxf(bb[3], (float)col);
        }
    }
    // 5. order-independent min/max reductions and the final counts
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        bb[0] = fminf(bb[0], __shfl_xor(bb[0], off, NC_WAVE));
        bb[1] = fmaxf(bb[1], __shfl_xor(bb[1], off, NC_WAVE));
        bb[2] = fminf(bb[2], __shfl_xor(bb[2], off, NC_WAVE));
        bb[3] = fmaxf(bb[3], __shfl_xor(bb[3], off, NC_WAVE));
        rh = fmaxf(rh, __shfl_xor(rh, off, NC_WAVE));
        rw = fmaxf(rw, __shfl_xor(rw, off, NC_WAVE));
    }
    const int lane = tid & 63, wave = tid >> 6;
    if (lane == 0) {
        red[0 * 16 + wave] = bb[0];
        red[1 * 16 + wave] = bb[1];
        red[2 * 16 + wave] = bb[2];
        red[3 * 16 + wave] = bb[3];
        red[4 * 16 + wave] = rh;
        red[5 * 16 + wave] = rw;
    }
    float cv[1] = {cnt};
    block_sum<1, kAdNT>(cv, peak_s);  // barriers also publish red[]
    if (tid == 0) {
        float a0 = hv, a1 = -1.f, a2 = wv, a3 = -1.f, a4 = 0.f, a5 = 0.f;
        for (int w_ = 0; w_ < kAdNT / 64; ++w_) {
            a0 = fminf(a0, red[w_]);
            a1 = fmaxf(a1, red[16 + w_]);
            a2 = fminf(a2, red[32 + w_]);
            a3 = fmaxf(a3, red[48 + w_]);
            a4 = fmaxf(a4, red[64 + w_]);
            a5 = fmaxf(a5, red[80 + w_]);
        }
        stats[0] = max(1, (int)a4);
        stats[1] = max(1, (int)a5);
        stats[2] = (int)cv[0];
        stats[3] = a1 >= 0.f ? 1 : 0;
        stats[4] = (int)a0;
        stats[5] = (int)a1 + 1;
        stats[6] = (int)a2;
        stats[7] = (int)a3 + 1;
    }
}

// ----------------------------------------------------------------------------------------
// Orchestration helpers
// ----------------------------------------------------------------------------------------

__global__ void k_inject(int B, int n_in, const float* __restrict__ in, int n_roi,
                         const int* __restrict__ src, float* __restrict__ roi) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)B * n_roi) return;
    const int b = (int)(q / n_roi), i = (int)(q % n_roi);
    const int e = src[i];
    roi[q] = e >= 0 ? in[(size_t)b * n_in + e] : 0.0f;
}

__global__ __launch_bounds__(1024) void k_mse(int n, const float* __restrict__ pred,
                                              const float* __restrict__ tgt,
                                              float* __restrict__ loss, float* __restrict__ g) {
    __shared__ float red[1024 / 64 + 1];
    const float inv_n = 1.0f / (float)n;
    float acc[1] = {0.f};
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float d = pred[i] - tgt[i];
        acc[0] += d * d;
        g[i] = 2.0f * d * inv_n;
    }
    block_sum<1, 1024>(acc, red);
    if (threadIdx.x == 0) loss[0] = acc[0] * inv_n;
}

// One workgroup walks the batch: byte = sum_j sat_u8(rint(out[b,j])) << (7-j), compared
// with the packed label; the matching count is exact in fp32 (B < 2^24), so the fp32
// batch mean and the running sum reproduce a sequential scan carry.
__global__ __launch_bounds__(1024) void k_packed_acc(int B, const float* __restrict__ out,
                                                     const uint8_t* __restrict__ y,
                                                     uint8_t* __restrict__ preds,
                                                     float* __restrict__ acc) {
    __shared__ float red[1024 / 64 + 1];
    float hit[1] = {0.f};
    for (int b = threadIdx.x; b < B; b += blockDim.x) {
        unsigned byte = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float r = rintf(out[(size_t)b * 8 + j]);
            const unsigned q = r > 0.f ? (r < 255.f ? (unsigned)r : 255u) : 0u;  // NaN -> 0
            byte += q << (7 - j);
        }
        byte &= 0xffu;
        if (preds) preds[b] = (uint8_t)byte;
        hit[0] += byte == (unsigned)y[b] ? 1.f : 0.f;
    }
    block_sum<1, 1024>(hit, red);
    if (threadIdx.x == 0) acc[0] = acc[0] + hit[0] / (float)B;
}

__global__ void k_adamw(int n, float* __restrict__ p, const float* __restrict__ g,
                        float* __restrict__ m, float* __restrict__ v,
                        const int* __restrict__ count, const float* __restrict__ lr, int n_lr,
                        float b1, float b2, float eps, float wd) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int c = count[0];
    const float rate = lr[c < n_lr ? c : n_lr - 1];
    const float t = (float)(c + 1);
    const float gi = g[i];
    const float mi = (1.0f - b1) * gi + b1 * m[i];
    const float vi = (1.0f - b2) * gi * gi + b2 * v[i];
    m[i] = mi;
    v[i] = vi;
    const float mh = mi / (1.0f - powf(b1, t));
    const float vh = vi / (1.0f - powf(b2, t));
    const float u = mh / (sqrtf(vh) + eps) + wd * p[i];
    p[i] = p[i] - rate * u;
}

// Gated filters (propagator.py:266-267): sigmoid of the raw filters, and the gradient's
// chain rule through it in place.
__global__ void k_gate_fwd(int n, const float* __restrict__ x, float* __restrict__ y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = nc_sigmoid(x[i]);
}

__global__ void k_gate_bwd(int n, const float* __restrict__ y, float* __restrict__ g) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) g[i] = g[i] * (y[i] * (1.0f - y[i]));
}

__global__ void k_count_inc(int* count) {
    if (threadIdx.x == 0 && blockIdx.x == 0) count[0] = count[0] + 1;
}

// ----------------------------------------------------------------------------------------
// The final universe (propagator.py:684-734): the last step's epilogue output on the active
// sub-ROI, the VALID border value final_act(B) * s_prob (zero without a VALID border)
// elsewhere, then the final activation over the whole grid; the output port is gathered
// from it by grid cell, so a port may lie anywhere on the grid.
// ----------------------------------------------------------------------------------------

struct UniverseArgs {
    nc_chip_desc c;
    int B, G, valid, fact;
    float slope;
    const float* parts;  // (G, B, h, w) direction-group partials of the ROI epilogue output
    const float* bfull;  // (H, W) cell biases
    const float* sprob;  // (H, W) Codd probabilities
};

// The activation's argument at (b, grid cell q); *roi says whether q is a sub-ROI cell.
NC_DEV float universe_pre(const UniverseArgs& a, int b, int q, bool* roi) {
    const int r = q / a.c.W, col = q % a.c.W;
    const int h = a.c.r1 - a.c.r0, w = a.c.c1 - a.c.c0;
    const int ri = r - a.c.pad_h - a.c.r0, ci = col - a.c.pad_w - a.c.c0;
    *roi = ri >= 0 && ri < h && ci >= 0 && ci < w;
    if (*roi) {
        const size_t plane = (size_t)a.B * h * w;
        const float* p = a.parts + (size_t)b * h * w + ri * w + ci;
        float v = 0.0f;
        for (int g = 0; g < a.G; ++g) v += p[g * plane];
        return v;
    }
    return a.valid ? nc_act(a.bfull[q], a.fact, a.slope) * a.sprob[q] : 0.0f;
}

// Threads [0, B*H*W) write the universe (when requested), threads past them the B*P port
// outputs, each evaluated from the same operands.
__global__ void k_universe_fwd(UniverseArgs a, int P, const int* __restrict__ cells,
                               float* __restrict__ univ, float* __restrict__ out) {
    const size_t HW = (size_t)a.c.H * a.c.W;
    const size_t nu = univ ? (size_t)a.B * HW : 0;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    bool roi;
    if (q < nu) {
        const int b = (int)(q / HW), cell = (int)(q % HW);
        univ[q] = nc_act(universe_pre(a, b, cell, &roi), a.fact, a.slope);
    } else if (q < nu + (size_t)a.B * P) {
        const size_t k = q - nu;
        const int b = (int)(k / P), p = (int)(k % P);
        out[k] = nc_act(universe_pre(a, b, cells[p], &roi), a.fact, a.slope);
    }
}

// Cotangent of the final cells at (b, q): the universe's own plus every port output read
// from q (head/next chain the ports by cell, in port order).
NC_DEV float universe_cot(int b, int q, size_t HW, int P, const int* head, const int* next,
                          const float* g_out, const float* g_univ) {
    float g = g_univ ? g_univ[(size_t)b * HW + q] : 0.0f;
    if (g_out)
        for (int p = head[q]; p >= 0; p = next[p]) g += g_out[(size_t)b * P + p];
    return g;
}

// Sub-ROI cells: g_roi (B, h, w) = cotangent * final_act'(pre).
__global__ void k_universe_bwd_roi(UniverseArgs a, int P, const int* __restrict__ head,
                                   const int* __restrict__ next, const float* __restrict__ g_out,
                                   const float* __restrict__ g_univ, float* __restrict__ g_roi) {
    const int h = a.c.r1 - a.c.r0, w = a.c.c1 - a.c.c0;
    const size_t n = (size_t)h * w;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)a.B * n) return;
    const int b = (int)(q / n), i = (int)(q % n);
    const int cell = (a.c.pad_h + a.c.r0 + i / w) * a.c.W + a.c.pad_w + a.c.c0 + i % w;
    bool roi;
    const float v = universe_pre(a, b, cell, &roi);
    float y;
    const float d = nc_act_d(v, a.fact, a.slope, &y);
    g_roi[q] = universe_cot(b, cell, (size_t)a.c.H * a.c.W, P, head, next, g_out, g_univ) * d;
}

// Border cells (VALID): the batch-summed cotangent through final_act(final_act(B) * s_prob)
// onto B and s_prob; zero on the sub-ROI cells.
__global__ void k_universe_bwd_border(UniverseArgs a, int P, const int* __restrict__ head,
                                      const int* __restrict__ next,
                                      const float* __restrict__ g_out,
                                      const float* __restrict__ g_univ,
                                      float* __restrict__ g_sprob, float* __restrict__ g_bfull) {
    const size_t HW = (size_t)a.c.H * a.c.W;
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (int)HW) return;
    bool roi;
    const float v = universe_pre(a, 0, q, &roi);
    float gs = 0.0f, gb = 0.0f;
    if (!roi) {
        float gsum = 0.0f;
        for (int b = 0; b < a.B; ++b) gsum += universe_cot(b, q, HW, P, head, next, g_out, g_univ);
        float y, ab;
        const float gv = gsum * nc_act_d(v, a.fact, a.slope, &y);
        const float dab = nc_act_d(a.bfull[q], a.fact, a.slope, &ab);
        gs = gv * ab;
        gb = gv * a.sprob[q] * dab;
    }
    g_sprob[q] = gs;
    g_bfull[q] = gb;
}

int chip_ok(const nc_chip_desc* c) {
    if (!c) return 0;
    if (c->H <= 0 || c->W <= 0 || c->kh <= 0 || c->kw <= 0 || c->M <= 0) return 0;
    if ((c->kh & 1) == 0 || (c->kw & 1) == 0) return 0;
    if (c->roi_h != c->H - 2 * c->pad_h || c->roi_w != c->W - 2 * c->pad_w) return 0;
    if (c->roi_h <= 0 || c->roi_w <= 0) return 0;
    if (c->r0 < 0 || c->r1 > c->roi_h || c->r0 >= c->r1) return 0;
    if (c->c0 < 0 || c->c1 > c->roi_w || c->c0 >= c->c1) return 0;
    // with a padded ROI (VALID) the sub-ROI's receptive field must stay inside the grid; with
    // none (SAME / CIRCULAR: the grid is the ROI) there is no border and the patch's cells
    // beyond the grid are never formed
    if ((c->pad_h > 0 || c->pad_w > 0) && (c->r1 + c->kh - 1 > c->H || c->c1 + c->kw - 1 > c->W))
        return 0;
    return 1;
}

}  // namespace

extern "C" {

int nc_version(void) { return NC_ABI_VERSION; }

const char* nc_strerror(int status) {
    switch (status) {
        case NC_OK: return "ok";
        case NC_ERR_INVALID_ARGUMENT: return "invalid argument";
        case NC_ERR_UNSUPPORTED: return "unsupported shape or configuration";
        case NC_ERR_WORKSPACE: return "workspace missing or too small";
        case NC_ERR_SCRATCH_LIMIT:
            return "shapes exceed the allocation-free entry point's scratch maximum";
        default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
    }
}

int nc_codd_fuse_fwd(void* stream, const nc_chip_desc* chip, const float* cell,
                     const uint8_t* io_mask, const uint8_t* out_weight_mask, int codd_mode,
                     float inv_tau, float active_threshold, int hard_pin_io, int act,
                     float neg_slope, int n_port, const int32_t* port_rc, float* w_eff,
                     float* s_eff, float* b_roi, float* border_patch, float* port_params,
                     float* s_prob, float* border_2d, float* w_pinned) {
    if (!chip_ok(chip) || !cell || !io_mask || !out_weight_mask || codd_mode < 0 ||
        codd_mode > 3 || act < 0 || act > 5 || n_port < 0 || (n_port > 0 && !port_rc) ||
        !w_eff || !s_eff || !b_roi || !border_patch || (n_port > 0 && !port_params))
        return NC_ERR_INVALID_ARGUMENT;
    const int n = chip->H * chip->W + n_port;
    hipLaunchKernelGGL(k_codd_fwd, dim3((n + 255) / 256), dim3(256), 0, nc_stream(stream), *chip,
                       cell, io_mask, out_weight_mask, codd_mode, inv_tau, active_threshold,
                       hard_pin_io, act, neg_slope, n_port, port_rc, w_eff, s_eff, b_roi,
                       border_patch, port_params, s_prob, border_2d, w_pinned);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_codd_fuse_bwd(void* stream, const nc_chip_desc* chip, const float* cell,
                     const uint8_t* io_mask, const uint8_t* out_weight_mask, int codd_mode,
                     float inv_tau, float active_threshold, int hard_pin_io, int act,
                     float neg_slope, int n_port, const int32_t* port_rc,
                     const int32_t* port_cell_start, const int32_t* port_cell_list,
                     const float* g_w_eff, const float* g_s_eff, const float* g_b_roi,
                     const float* g_border_patch, const float* g_port_params,
                     const float* g_s_prob, const float* g_b_full, float* g_cell) {
    if (!chip_ok(chip) || !cell || !io_mask || !out_weight_mask || codd_mode < 0 ||
        codd_mode > 3 || act < 0 || act > 5 || n_port < 0 || (n_port > 0 && !port_rc) ||
        !g_cell || (!port_cell_start != !port_cell_list))
        return NC_ERR_INVALID_ARGUMENT;
    const int n = chip->H * chip->W;
    hipLaunchKernelGGL(k_codd_bwd, dim3((n + 255) / 256), dim3(256), 0, nc_stream(stream), *chip,
                       cell, io_mask, out_weight_mask, codd_mode, inv_tau, active_threshold,
                       hard_pin_io, act, neg_slope, n_port, port_rc, port_cell_start,
                       port_cell_list, g_w_eff, g_s_eff, g_b_roi,
                       g_border_patch, n_port > 0 ? g_port_params : nullptr, g_s_prob,
                       g_b_full, g_cell);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_adaptive_stats(void* stream, const nc_chip_desc* chip, const float* cell,
                      const float* filters, const uint8_t* io_mask_roi, const float* act_roi,
                      int margin_h, int margin_w, float salience_threshold, float bias_threshold,
                      float filter_threshold, float activity_threshold, int32_t* stats,
                      uint8_t* dilated) {
    if (!chip_ok(chip) || !cell || !filters || !io_mask_roi || !stats || !dilated ||
        margin_h < 0 || margin_w < 0)
        return NC_ERR_INVALID_ARGUMENT;
    const size_t N = (size_t)chip->roi_h * chip->roi_w;
    if (2 * N > 65536) return NC_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(k_adaptive, dim3(1), dim3(kAdNT), 2 * N, nc_stream(stream), *chip, cell,
                       filters, io_mask_roi, act_roi, margin_h, margin_w, salience_threshold,
                       bias_threshold, filter_threshold, activity_threshold, stats, dilated);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_inject_roi(void* stream, int B, int n_in, const float* inputs, int n_roi,
                  const int32_t* src, float* roi) {
    if (B <= 0 || n_in <= 0 || n_roi <= 0 || !inputs || !src || !roi)
        return NC_ERR_INVALID_ARGUMENT;
    const size_t n = (size_t)B * n_roi;
    hipLaunchKernelGGL(k_inject, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       nc_stream(stream), B, n_in, inputs, n_roi, src, roi);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_mse_loss(void* stream, int n, const float* pred, const float* target, float* loss,
                float* g_pred) {
    if (n <= 0 || !pred || !target || !loss || !g_pred) return NC_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_mse, dim3(1), dim3(1024), 0, nc_stream(stream), n, pred, target, loss,
                       g_pred);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_packed_accuracy(void* stream, int B, int n_out, const float* out,
                       const uint8_t* y_packed, uint8_t* preds_packed, float* acc) {
    if (B <= 0 || n_out != 8 || !out || !y_packed || !acc) return NC_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_packed_acc, dim3(1), dim3(1024), 0, nc_stream(stream), B, out, y_packed,
                       preds_packed, acc);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_adamw_step(void* stream, int n, float* p, const float* g, float* m, float* v,
                  int32_t* count, const float* lr, int n_lr, float b1, float b2, float eps,
                  float weight_decay) {
    if (n <= 0 || n_lr <= 0 || !p || !g || !m || !v || !count || !lr)
        return NC_ERR_INVALID_ARGUMENT;
    hipStream_t st = nc_stream(stream);
    hipLaunchKernelGGL(k_adamw, dim3((n + 255) / 256), dim3(256), 0, st, n, p, g, m, v, count, lr,
                       n_lr, b1, b2, eps, weight_decay);
    NC_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_count_inc, dim3(1), dim3(64), 0, st, count);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_filter_gate_fwd(void* stream, int n, const float* filters, float* gated) {
    if (n <= 0 || !filters || !gated) return NC_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_gate_fwd, dim3((n + 255) / 256), dim3(256), 0, nc_stream(stream), n,
                       filters, gated);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_filter_gate_bwd(void* stream, int n, const float* gated, float* g_filters) {
    if (n <= 0 || !gated || !g_filters) return NC_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(k_gate_bwd, dim3((n + 255) / 256), dim3(256), 0, nc_stream(stream), n,
                       gated, g_filters);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_universe_fwd(void* stream, const nc_chip_desc* chip, int B, int G, int valid_border,
                    int final_act, float neg_slope, const float* parts, const float* b_full,
                    const float* s_prob, int n_port, const int32_t* port_cells, float* universe,
                    float* out) {
    if (!chip_ok(chip) || B <= 0 || G <= 0 || final_act < 0 || final_act > 5 || !parts ||
        n_port < 0 || (n_port > 0 && (!port_cells || !out)) || (!universe && n_port == 0) ||
        (valid_border && (!b_full || !s_prob)))
        return NC_ERR_INVALID_ARGUMENT;
    const UniverseArgs a{*chip, B, G, valid_border != 0, final_act, neg_slope, parts, b_full,
                         s_prob};
    const size_t n = (universe ? (size_t)B * chip->H * chip->W : 0) + (size_t)B * n_port;
    hipLaunchKernelGGL(k_universe_fwd, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       nc_stream(stream), a, n_port, port_cells, universe, out);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

int nc_universe_bwd(void* stream, const nc_chip_desc* chip, int B, int G, int valid_border,
                    int final_act, float neg_slope, const float* parts, const float* b_full,
                    const float* s_prob, int n_port, const int32_t* port_head,
                    const int32_t* port_next, const float* g_out, const float* g_universe,
                    float* g_roi, float* g_s_prob, float* g_b_full) {
    if (!chip_ok(chip) || B <= 0 || G <= 0 || final_act < 0 || final_act > 5 || !parts ||
        n_port < 0 || (n_port > 0 && g_out && (!port_head || !port_next)) || !g_roi ||
        (valid_border && (!b_full || !s_prob || !g_s_prob || !g_b_full)))
        return NC_ERR_INVALID_ARGUMENT;
    const UniverseArgs a{*chip, B, G, valid_border != 0, final_act, neg_slope, parts, b_full,
                         s_prob};
    const int P = g_out ? n_port : 0;
    const size_t n = (size_t)B * (chip->r1 - chip->r0) * (chip->c1 - chip->c0);
    hipLaunchKernelGGL(k_universe_bwd_roi, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       nc_stream(stream), a, P, port_head, port_next, g_out, g_universe, g_roi);
    NC_CHECK_LAUNCH();
    if (valid_border) {
        const int hw = chip->H * chip->W;
        hipLaunchKernelGGL(k_universe_bwd_border, dim3((hw + 255) / 256), dim3(256), 0,
                           nc_stream(stream), a, P, port_head, port_next, g_out, g_universe,
                           g_s_prob, g_b_full);
        NC_CHECK_LAUNCH();
    }
    return NC_OK;
}

int nc_step_prologue(void* stream, const nc_chip_desc* chip, const float* cell,
                     const uint8_t* io_mask, const uint8_t* out_weight_mask, int codd_mode,
                     float inv_tau, float active_threshold, int hard_pin_io, int act,
                     float neg_slope, int n_port, const int32_t* port_rc, float* w_eff,
                     float* s_eff, float* b_roi, float* border_patch, float* port_params,
                     float* s_prob, int B, int n_in, const float* inputs, int n_roi,
                     const int32_t* src, float* roi) {
    if (!chip_ok(chip) || !cell || !io_mask || !out_weight_mask || codd_mode < 0 ||
        codd_mode > 3 || act < 0 || act > 5 || n_port < 0 || (n_port > 0 && !port_rc) ||
        !w_eff || !s_eff || !b_roi || !border_patch || (n_port > 0 && !port_params) || B <= 0 ||
        n_in <= 0 || n_roi <= 0 || !inputs || !src || !roi)
        return NC_ERR_INVALID_ARGUMENT;
    const InjectArgs ia{B, n_in, n_roi, inputs, src, roi};
    const size_t n = (size_t)chip->H * chip->W + n_port + (size_t)B * n_roi;
    hipLaunchKernelGGL(k_prologue, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       nc_stream(stream), *chip, cell, io_mask, out_weight_mask, codd_mode,
                       inv_tau, active_threshold, hard_pin_io, act, neg_slope, n_port, port_rc,
                       w_eff, s_eff, b_roi, border_patch, port_params, s_prob, ia);
    NC_CHECK_LAUNCH();
    return NC_OK;
}

}  // extern "C"

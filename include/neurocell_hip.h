/*
 * neurocell_hip.h - C ABI of the MI355X (gfx950 / CDNA4) Neurocell v2 VNN propagation step.
 *
 * One extern "C" entry point per kernel family of the reference's operator layer.  Every
 * entry point:
 *   - takes a hipStream_t as `void* stream` (NULL = the default stream);
 *   - takes device pointers only (row-major, contiguous; NCHW planes; complex spectra as
 *     interleaved float pairs (re, im) in (fft_h, fft_w/2+1) row-major layout);
 *   - never allocates, never synchronises the host, and never copies host<->device, so a
 *     caller may capture it in a HIP graph; scratch comes in through (ws, ws_bytes), sized
 *     by the matching *_workspace_size() query;
 *   - returns NC_OK (0) or a negative NC_ERR_* status (or a positive hipError_t when a
 *     launch fails); it never throws across the ABI;
 *   - is deterministic: every reduction (over pixels, directions M, batch B or FFT bins)
 *     runs in a fixed order, with no atomics.
 *
 * Citations name the reference operator (path:line in shakes76/neurocell-v2) whose forward or
 * custom-VJP rule the entry point replaces.
 */
#ifndef NEUROCELL_HIP_H_
#define NEUROCELL_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NC_ABI_VERSION 1

/* Status codes. */
#define NC_OK 0
#define NC_ERR_INVALID_ARGUMENT (-1)
#define NC_ERR_UNSUPPORTED (-2)
#define NC_ERR_WORKSPACE (-3)
#define NC_ERR_SCRATCH_LIMIT (-4) /* shapes beyond the allocation-free scratch maximum */

/* Bytes of the file-scope device scratch behind the allocation-free entry points (one array
 * per GPU, held until the process ends). */
#define NC_NOALLOC_SCRATCH_BYTES (16u << 20)

/* Activation ids: kernels_pallas.py:76-99 (_resolve_activation_spec). */
#define NC_ACT_IDENTITY 0
#define NC_ACT_TANH 1
#define NC_ACT_SIGMOID 2
#define NC_ACT_RELU 3
#define NC_ACT_LEAKY_RELU 4
#define NC_ACT_GELU 5

/* Codd modes: params.py:23-28 (SUPPORTED_CODD_MODES, same order). */
#define NC_CODD_CONTINUOUS 0
#define NC_CODD_ANNEALED 1
#define NC_CODD_STE_BINARY 2
#define NC_CODD_STE_TERNARY 3

/*
 * Static chip geometry for the pre-step fusion (topology.py:109-284 ChipTopology2D plus the
 * adaptive crop of adaptive_mask.py:164-197).  The active sub-ROI is [r0, r1) x [c0, c1) in
 * ROI coordinates; (0, roi_h, 0, roi_w) when uncropped.
 */
typedef struct nc_chip_desc {
    int32_t H, W;          /* grid */
    int32_t kh, kw;        /* Green's-filter size (odd) */
    int32_t M;             /* directions */
    int32_t pad_h, pad_w;  /* ROI offset in the grid (VALID: (kh-1)/2, (kw-1)/2) */
    int32_t roi_h, roi_w;  /* full ROI */
    int32_t r0, r1, c0, c1;/* active sub-ROI */
} nc_chip_desc;

int nc_version(void);
const char* nc_strerror(int status);

/* ---------------- piece 1: pre-step Codd fusion ---------------------------------------- */

/*
 * compute_codd_state_probs + precompute_step_params forward (params.py:31-80, 220-322) and
 * the border template of propagator.py:355-361.
 * In : cell (3,H,W) = [W, B, S_raw]; io_mask, out_weight_mask (H,W) u8; port_rc (2,P) int32
 *      ROI (uncropped) row then column indices of the P output-port cells.
 * Out: w_eff, s_eff, b_roi (h,w) for the active sub-ROI (h = r1-r0, w = c1-c0);
 *      border_patch (h+kh-1, w+kw-1) = act(B)*s_prob with the ROI zeroed, cut at grid
 *      offset (r0, c0) (with pad 0, the SAME / CIRCULAR modes, the ROI is the whole grid:
 *      the patch is zero on the grid and its cells beyond the grid are left unwritten); port_params (3,P) = [w_eff_out, s_eff_out, b_out]; optional (NULL
 *      to skip) full-grid s_prob, border_2d = act(B)*s_prob and w_pinned, each (H,W).
 * inv_tau is 1/max(tau, 1e-4) rounded to float32 (params.py:63).
 */
int nc_codd_fuse_fwd(void* stream, const nc_chip_desc* chip, const float* cell,
                     const uint8_t* io_mask, const uint8_t* out_weight_mask, int codd_mode,
                     float inv_tau, float active_threshold, int hard_pin_io, int act,
                     float neg_slope, int n_port, const int32_t* port_rc, float* w_eff,
                     float* s_eff, float* b_roi, float* border_patch, float* port_params,
                     float* s_prob, float* border_2d, float* w_pinned);

/*
 * A step's prologue in one launch: nc_codd_fuse_fwd (without its border_2d and w_pinned
 * outputs) and nc_inject_roi(B, n_in, inputs, n_roi, src, roi), which are independent.
 * Same arguments and results as the two calls; src entries must lie in [-1, n_in).
 * No reference counterpart of its own: it saves one launch of the pre-step work of
 * propagator.py:252-263 and :344-352.
 */
int nc_step_prologue(void* stream, const nc_chip_desc* chip, const float* cell,
                     const uint8_t* io_mask, const uint8_t* out_weight_mask, int codd_mode,
                     float inv_tau, float active_threshold, int hard_pin_io, int act,
                     float neg_slope, int n_port, const int32_t* port_rc, float* w_eff,
                     float* s_eff, float* b_roi, float* border_patch, float* port_params,
                     float* s_prob, int B, int n_in, const float* inputs, int n_roi,
                     const int32_t* src, float* roi);

/*
 * Reverse of nc_codd_fuse_fwd (the autodiff of params.py:220-322 and of the STE forms of
 * params.py:58-80).  Any gradient input may be NULL (zero).  g_s_prob and g_b_full (H,W) are
 * full-grid gradients with respect to s_prob (the reverse of the optional s_prob output) and
 * to the cell biases B themselves (the final universe's border term).  Writes g_cell (3,H,W).
 * port_cell_start (roi_h*roi_w + 1) / port_cell_list (n_port), both NULL or both given: the
 * port indices by ROI cell (cell o's ports are list[start[o] .. start[o+1]), in increasing
 * port order), so each cell gathers its port-parameter gradients without scanning port_rc;
 * the sums are the same either way.
 */
int nc_codd_fuse_bwd(void* stream, const nc_chip_desc* chip, const float* cell,
                     const uint8_t* io_mask, const uint8_t* out_weight_mask, int codd_mode,
                     float inv_tau, float active_threshold, int hard_pin_io, int act,
                     float neg_slope, int n_port, const int32_t* port_rc,
                     const int32_t* port_cell_start, const int32_t* port_cell_list,
                     const float* g_w_eff, const float* g_s_eff, const float* g_b_roi,
                     const float* g_border_patch, const float* g_port_params,
                     const float* g_s_prob, const float* g_b_full, float* g_cell);

/*
 * The final universe and the full-grid output port (propagator.py:684-734, with
 * _extract_output_from_full_grid :194-206): the path taken for return_universe=True and for
 * an output port outside the VALID ROI (topology.py allow_border_output / full-grid ports).
 * parts (G,B,h,w) are the direction-group partials of the last step's ROI epilogue run with
 * the final activation (nc_fftconv_epilogue_fwd with act = final_act); their sum is the
 * sub-ROI's pre-activation.  Every other grid cell takes final_act(B) * s_prob when
 * valid_border (VALID mode, b_full = cell[1] and s_prob from nc_codd_fuse_fwd), else 0.
 * universe (B,H,W) = final_act(pre) over the grid (NULL to skip); out (B,P) = the universe
 * at port_cells (P grid-flat cell indices, each in [0, H*W)).
 */
int nc_universe_fwd(void* stream, const nc_chip_desc* chip, int B, int G, int valid_border,
                    int final_act, float neg_slope, const float* parts, const float* b_full,
                    const float* s_prob, int n_port, const int32_t* port_cells, float* universe,
                    float* out);

/*
 * Reverse of nc_universe_fwd.  The final cells' cotangent is g_universe (B,H,W; NULL = 0)
 * plus g_out (B,P; NULL = 0) added at each port's cell: port_head (H*W) holds the first port
 * at each cell or -1, port_next (P) the next port at the same cell or -1 (an acyclic chain in
 * port order).  Writes g_roi (B,h,w), the cotangent of the ROI epilogue's output (feed it to
 * nc_epilogue_bwd_parts with act = final_act); with valid_border also g_s_prob and g_b_full
 * (H,W) for nc_codd_fuse_bwd (zero on the sub-ROI cells).
 */
int nc_universe_bwd(void* stream, const nc_chip_desc* chip, int B, int G, int valid_border,
                    int final_act, float neg_slope, const float* parts, const float* b_full,
                    const float* s_prob, int n_port, const int32_t* port_head,
                    const int32_t* port_next, const float* g_out, const float* g_universe,
                    float* g_roi, float* g_s_prob, float* g_b_full);

/*
 * gated_filters (propagator.py:266-267): gated (n) = sigmoid(filters); the reverse turns the
 * gradient with respect to the gated filters, g_filters (n), into the gradient with respect to
 * the raw filters in place: g *= gated * (1 - gated).
 */
int nc_filter_gate_fwd(void* stream, int n, const float* filters, float* gated);
int nc_filter_gate_bwd(void* stream, int n, const float* gated, float* g_filters);

/* ---------------- piece 2: Green's-function convolution (spectral) -------------------- */

/*
 * precompute_filter_rfft2 / hoist_filter_rfft2(_nopad) forward (kernels_greens.py:240-259,
 * kernels_pallas.py:1582-1604): ghat (M, fft_h, fft_w/2+1) complex = rfft2 of the flipped
 * filters (M,1,kh,kw).
 */
int nc_filter_spectrum_fwd(void* stream, int M, int kh, int kw, int fft_h, int fft_w,
                           const float* filters, float* ghat);

/*
 * rfft2_unshifted_filter_grad_to_oihw (kernels_pallas.py:1558-1579), the backward of
 * hoist_filter_rfft2_nopad: irfft2(dghat) rolled by (shift_h, shift_w), cropped to
 * (kh,kw) and flipped.  g_filters (M,1,kh,kw) is overwritten, or added to when accumulate.
 * dghat follows the reference's (JAX) complex-cotangent convention, dL/dRe - i dL/dIm;
 * conj_in != 0 takes it in the conjugate (PyTorch autograd) convention instead.
 */
int nc_filter_spectrum_bwd(void* stream, int M, int kh, int kw, int fft_h, int fft_w,
                           int shift_h, int shift_w, const float* dghat, float* g_filters,
                           int accumulate, int conj_in);

/*
 * The end of a reverse pass with a border term in one launch: nc_filter_spectrum_bwd
 * (dghat -> g_filters) and the border patch's gradient of nc_fftconv_bwd_hat without dghat
 * (g_patch (hp, wp) = irfft2(sum over m of gz_hat_m * conj(ghat_m)) rolled by
 * (pshift_h, pshift_w), cropped): the patch spectrum's reduction over m, then one launch for
 * all M + 1 inverse transforms.  ws: fft_h * (fft_w/2+1) complex values.
 * No counterpart in the reference.
 */
int nc_filter_patch_bwd(void* stream, int M, int kh, int kw, int fft_h, int fft_w,
                        int shift_h, int shift_w, const float* dghat, float* g_filters,
                        int accumulate, int conj_in, int hp, int wp, int pshift_h, int pshift_w,
                        const float* gz_hat, const float* ghat, float* g_patch, void* ws,
                        size_t ws_bytes);

/*
 * Overlap-save spectral cross-correlation forward: conv2d_pruned_rfft_roi_step /
 * conv2d_roi_rfft_step forward (kernels_pallas.py:1759-1791, kernels_greens.py:316-360) and,
 * with pad = (kh-1, kw-1), conv2d_valid_rfft_precomputed (kernels_greens.py:403-425) and the
 * hoisted border conv (propagator.py:362-366).
 * x (B, hin, win) real, placed at the spectral origin; z (B, M, hout, wout) =
 * irfft2(rfft2(x) * ghat)[pad_h : pad_h+hout, pad_w : pad_w+wout].  xhat (B, fft_h,
 * fft_w/2+1) complex receives the cell spectra (the saved cell_freq residual); it is required
 * (the correlation reads it back).
 * Supported spectral grids: fft_h, fft_w both in {16, 32, 64} (wavefront transforms) or
 * both in {64, 128, 256} (workgroup transforms over LDS segments).
 * The output window is read modulo the grid (pad_h < fft_h, hout <= fft_h, and likewise
 * for w): with the grid equal to the plane, hin = hout = fft_h, this is the circular
 * correlation of the reference's CIRCULAR padding mode (propagator.py:284-300).
 */
int nc_fftconv_fwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int pad_h,
                   int pad_w, int fft_h, int fft_w, const float* x, const float* ghat, float* z,
                   float* xhat);

/*
 * nc_fftconv_fwd with xhat_add (fft_h, fft_w/2+1) complex added to every sample's spectrum
 * before the correlation (NULL: none); xhat receives the sums.  With xhat_add = the
 * nc_plane_spectrum of the border patch shifted by (pad_h - (kh-1), pad_w - (kw-1)) mod the
 * grid, z = the ROI correlation plus the hoisted border conv delta (propagator.py:362-366,
 * 425-441) in one pass, and the reverse through nc_fftconv_bwd_ex carries the border's dG.
 * No counterpart in the reference (which adds delta to every step's conv output).
 */
int nc_fftconv_fwd_ex(void* stream, int B, int M, int hin, int win, int hout, int wout,
                      int pad_h, int pad_w, int fft_h, int fft_w, const float* x,
                      const float* xhat_add, const float* ghat, float* z, float* xhat);

/*
 * nc_fftconv_fwd_ex with x given as n_parts partial planes x_parts (n_parts, B, hin, win):
 * x = their sum in increasing order (the parts of nc_epilogue_fwd_parts).
 */
int nc_fftconv_fwd_parts(void* stream, int B, int M, int hin, int win, int hout, int wout,
                         int pad_h, int pad_w, int fft_h, int fft_w, const float* x_parts,
                         int n_parts, const float* xhat_add, const float* ghat, float* z,
                         float* xhat);

/*
 * Half-spectra (nplanes, fft_h, fft_w/2+1) complex of real (hin, win) planes placed at the
 * origin of the spectral grid and circularly shifted by (shift_h, shift_w)
 * (0 <= shift < grid): rfft2 times the phase ramp W^(kh*shift_h) W^(kw*shift_w), from exact
 * table twiddles.  Supported grids as nc_fftconv_fwd.  No counterpart in the reference.
 */
int nc_plane_spectrum(void* stream, int nplanes, int hin, int win, int fft_h, int fft_w,
                      int shift_h, int shift_w, const float* x, float* xhat);

/* One job of nc_plane_spectra: the half-spectra of nplanes real (hin, win) planes. */
typedef struct nc_spectrum_job {
    const float* x;       /* (nplanes, hin, win) real planes */
    float* xhat;          /* (nplanes, fft_h, fft_w/2+1) complex out */
    const float* add;     /* NULL, or one (fft_h, fft_w/2+1) spectrum added to each plane's */
    int nplanes, hin, win;
    int flip;             /* planes read rotated by 180 degrees: the filter spectra */
    int shift_h, shift_w; /* circular shift on the grid, as nc_plane_spectrum; 0 for none */
} nc_spectrum_job;

/*
 * Up to 4 independent spectrum jobs in one call: each job is nc_filter_spectrum_fwd (flip),
 * nc_plane_spectrum (shift), the spectra step of nc_fftconv_fwd_ex (add) or a plain rfft2 -
 * at most one of flip / add / shift per job.  On the 64-wide lane-pair grids all jobs run in
 * one launch.  No counterpart in the reference (which computes each spectrum in its own op).
 */
int nc_plane_spectra(void* stream, int fft_h, int fft_w, int n_jobs, const nc_spectrum_job* jobs);

/*
 * The correlation step of nc_fftconv_fwd from given cell spectra: z (B, M, hout, wout) =
 * irfft2(xhat_b * ghat_m)[pad_h : pad_h+hout, pad_w : pad_w+wout] (kernels_pallas.py:
 * 1779-1791), xhat (B, fft_h, fft_w/2+1) complex as nc_fftconv_fwd writes it.
 */
int nc_spectral_correlate(void* stream, int B, int M, int hout, int wout, int pad_h, int pad_w,
                          int fft_h, int fft_w, const float* xhat, const float* ghat, float* z);

/*
 * rfft2_pruned (kernels_greens.py:25-44) is nc_plane_spectrum with shift (0, 0): the
 * half-spectra of real planes zero-padded to the grid.
 *
 * irfft2_pruned (kernels_greens.py:47-66): out (nplanes, hout, wout) = irfft2(xhat)[pad_h :
 * pad_h+hout, pad_w : pad_w+wout] (the window read modulo the grid), xhat (nplanes, fft_h,
 * fft_w/2+1) complex.  As a real inverse transform does, only the Hermitian parts of the DC
 * and Nyquist columns enter.  Grids as nc_fftconv_fwd; ws sized by
 * nc_irfft2_pruned_workspace_size.
 */
size_t nc_irfft2_pruned_workspace_size(int nplanes, int fft_h, int fft_w);
int nc_irfft2_pruned(void* stream, int nplanes, int hout, int wout, int pad_h, int pad_w,
                     int fft_h, int fft_w, const float* xhat, float* out, void* ws,
                     size_t ws_bytes);

/*
 * Elementwise map of nplanes half-spectra (fft_h, fft_w/2+1) complex, any power-of-two grid:
 * out = phase(shift) * scale * H(conj_in ? conj(in) : in), where H replaces the DC and Nyquist
 * columns by their Hermitian parts along the column when herm_edges ((v[k] + conj(v[-k]))/2;
 * out must not alias in then), scale is edge_scale on those two columns and interior_scale
 * elsewhere, and phase(shift) = W^(kh*shift_h) W^(kw*shift_w), W = exp(-2 pi i / grid) (the
 * spectrum of the plane circularly shifted by shift).  in == NULL maps the constant 1.
 * It turns the unshifted Plancherel cotangent into the shifted one of conv2d_roi_rfft_step
 * (kernels_greens.py:363-400; the padded-gz spectrum is the unpadded one times the phase of
 * the pad) and gives the adjoints of rfft2_pruned / irfft2_pruned their column weights.
 */
int nc_spectrum_map(void* stream, int nplanes, int fft_h, int fft_w, int shift_h, int shift_w,
                    int herm_edges, float edge_scale, float interior_scale, int conj_in,
                    const float* in, float* out);

/*
 * Direct (spatial) correlation for small filters (kh * kw <= 64, M <= 64, plane widths <=
 * 256): conv2d_batched_nchw and the reference's small-kernel path (kernels_greens.py:177-217,
 * 84-123; propagator.py:373-386, 521-540), where a spectral grid would be mostly padding.
 *   z[b, m, i, j] = sum over u < kh, v < kw of x[b, i + oh + u, j + ow + v] * G[m, u, v]
 * x (n_parts, B, hin, win): the sum of n_parts partial planes (1 for a plain input), zero
 * outside the plane, or read modulo it when `circular` (then hin = hout, win = wout: the
 * CIRCULAR padding mode).  (oh, ow) = (-(kh-1)/2, -(kw-1)/2) gives the SAME ROI step, (0, 0)
 * a VALID correlation.  filters (M, 1, kh, kw), z (B, M, hout, wout).
 */
int nc_direct_conv_fwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int oh,
                       int ow, int kh, int kw, int circular, const float* x, int n_parts,
                       const float* filters, float* z);

/*
 * 1 when the direct correlation runs at these shapes (kh * kw <= 64, M <= 64, planes up to
 * 256 wide and each kernel's one-row band within the workgroup's LDS; with reverse also the
 * reverse kernels'), else 0.  Host logic choosing between it and the spectral path
 * (propagator.py:373-386 takes the direct conv for kh * kw <= 64).
 */
int nc_direct_conv_fits(int M, int hin, int win, int hout, int wout, int kh, int kw,
                        int circular, int reverse);

/* Rows of the filter-gradient partials nc_direct_conv_bwd writes at these shapes. */
int nc_direct_conv_dg_partials(int B, int M, int hout, int wout, int kh, int kw);

/*
 * Reverse of nc_direct_conv_fwd for the output cotangent gz (B, M, hout, wout): dx (B, hin,
 * win) when need_dx (the correlation's adjoint; dx may be NULL otherwise) and the filter
 * gradient as nc_direct_conv_dg_partials(...) partial rows dg_parts (rows, M * kh * kw), each
 * a fixed-order sum over one band of one sample's pixels; their sum (nc_rows_sum) is
 * dG (M, 1, kh, kw).  kernels_greens.py:84-123 (conv2d_grouped_filter_grad) for the gradient.
 */
int nc_direct_conv_bwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int oh,
                       int ow, int kh, int kw, int circular, const float* gz, const float* x,
                       int n_parts, const float* filters, int need_dx, float* dx,
                       float* dg_parts);

/* Workspace bytes needed by nc_fftconv_bwd for these shapes. */
size_t nc_fftconv_bwd_workspace_size(int B, int M, int fft_h, int fft_w);

/*
 * Unshifted Plancherel backward of the spectral correlation (kernels_pallas.py:1794-1821);
 * on the 64-wide grids M <= 64 (NC_ERR_UNSUPPORTED above, as the epilogues):
 * ghat_g = rfft2(gz) at the origin;
 *   dx = irfft2(sum_m ghat_g * conj(ghat)) rolled by (pad_h, pad_w), cropped (hin, win)
 *        (written only when need_dx; dx may be NULL otherwise);
 *   dghat = sum_b ghat_g * conj(xhat)   (M, fft_h, fft_w/2+1) complex, overwritten or added
 *        to when accumulate - the B-reduction runs in the frequency domain, in fixed order;
 *        conj_dghat != 0 writes its conjugate (the PyTorch autograd convention).
 */
int nc_fftconv_bwd(void* stream, int B, int M, int hin, int win, int hout, int wout, int pad_h,
                   int pad_w, int fft_h, int fft_w, const float* gz, const float* xhat,
                   const float* ghat, int need_dx, float* dx, float* dghat, int accumulate,
                   int conj_dghat, void* ws, size_t ws_bytes);

/*
 * nc_fftconv_bwd that also forms gz_hat_sum (M, fft_h, fft_w/2+1) complex = sum_b rfft2(gz_b)
 * at the origin (overwritten, or added to when sum_accumulate; NULL skips it): the spectra of
 * the batch-summed cotangent, which is the border cotangent sum_b gz of the hoisted border
 * conv (propagator.py:362-366, the gdb of nc_epilogue_bwd / nc_port_bwd) in the frequency
 * domain.  It is summed in the same pass as dghat, so the cotangent planes are not read again.
 * No counterpart in the reference (which differentiates the border conv through JAX).
 */
int nc_fftconv_bwd_ex(void* stream, int B, int M, int hin, int win, int hout, int wout,
                      int pad_h, int pad_w, int fft_h, int fft_w, const float* gz,
                      const float* xhat, const float* ghat, int need_dx, float* dx, float* dghat,
                      int accumulate, int conj_dghat, float* gz_hat_sum, int sum_accumulate,
                      void* ws, size_t ws_bytes);

/*
 * nc_fftconv_bwd at B = 1 with the cotangent given by its spectra gz_hat (M, fft_h,
 * fft_w/2+1) complex (e.g. the gz_hat_sum of nc_fftconv_bwd_ex): the backward of the hoisted
 * border conv (propagator.py:362-366) without its cotangent planes.
 *   dx = irfft2(sum_m gz_hat_m * conj(ghat_m)) rolled by (pad_h, pad_w), cropped (hin, win);
 *   dghat (+)= gz_hat * conj(xhat) when dghat is not NULL (xhat: the (fft_h, fft_w/2+1)
 *   input spectrum; conj_dghat as in nc_fftconv_bwd).
 * ws: at least fft_h*(fft_w/2+1)*8 bytes (nc_fftconv_bwd_workspace_size(1, ...) suffices).
 */
int nc_fftconv_bwd_hat(void* stream, int M, int hin, int win, int pad_h, int pad_w, int fft_h,
                       int fft_w, const float* gz_hat, const float* xhat, const float* ghat,
                       float* dx, float* dghat, int accumulate, int conj_dghat, void* ws,
                       size_t ws_bytes);

/*
 * The number of partial rows nc_fftconv_bwd_parts writes per output at these shapes (its
 * sample chunks; on the large grids the reduction's sample slices, enough to give it ~512
 * workgroups).
 */
int nc_fftconv_bwd_partials(int B, int M, int fft_h, int fft_w);

/*
 * nc_fftconv_bwd_ex leaving the sample-chunk partials of dghat and gz_hat_sum unsummed:
 * dghat_parts and gz_hat_sum_parts are row stacks (nparts, M, fft_h, fft_w/2+1) complex,
 * nparts = nc_fftconv_bwd_partials(B, M, fft_h, fft_w); each call writes its rows (or adds to
 * them, accumulate / sum_accumulate, conjugated per row with conj_dghat), so a d-step reverse
 * pass sums its steps row by row and one nc_rows_sum adds the rows at its end: no chunk-sum
 * launch per step.
 * No counterpart in the reference.
 */
int nc_fftconv_bwd_parts(void* stream, int B, int M, int hin, int win, int hout, int wout,
                         int pad_h, int pad_w, int fft_h, int fft_w, const float* gz,
                         const float* xhat, const float* ghat, int need_dx, float* dx,
                         float* dghat_parts, int accumulate, int conj_dghat,
                         float* gz_hat_sum_parts, int sum_accumulate, void* ws, size_t ws_bytes);


/*
 * One reverse step of a hidden layer as one operation: nc_epilogue_bwd_parts (has_border = 0,
 * hidden planes h x w) on gy, then nc_fftconv_bwd_parts on the gz it gives (hout = h, wout =
 * w) - kernels_pallas.py:869-1064 followed by 1794-1821.  On the 128- and 256-point grids
 * with planes above 8192 pixels the cotangent spectra's first transform pass forms gz from
 * z, gy, the plane statistics and the epilogue's (c1, c2) sums as it reads them (the same
 * arithmetic as the epilogue's own last stage), so gz is neither stored nor read back and may
 * be NULL; elsewhere gz (B, M, h, w) is required and the two entries run in turn.  Results as
 * the two calls.  ws_epi / ws_fc: the two entries' workspaces (nc_epilogue_workspace_size,
 * nc_fftconv_bwd_workspace_size), distinct.  No counterpart in the reference.
 */
int nc_epilogue_fftconv_bwd_parts(void* stream, int B, int M, int h, int w, int act,
                                  float neg_slope, const float* z, const float* w_eff,
                                  const float* s_eff, const float* b_roi, const float* mean,
                                  const float* rstd, const float* gy, float* gz, float* pg_rows,
                                  size_t plane_stride, int hin, int win, int pad_h, int pad_w,
                                  int fft_h, int fft_w, const float* xhat, const float* ghat,
                                  int need_dx, float* dx, float* dghat_parts, int accumulate,
                                  int conj_dghat, float* gz_hat_sum_parts, int sum_accumulate,
                                  void* ws_epi, size_t ws_epi_bytes, void* ws_fc,
                                  size_t ws_fc_bytes);

/* ---------------- piece 3: hidden-step epilogue and output-port epilogue --------------- */

/*
 * Workspace bytes for nc_epilogue_fwd / nc_epilogue_bwd / nc_port_fwd / nc_port_bwd at these
 * shapes (partial results of the workgroups that share a sample, tile statistics, per-sample
 * parameter-gradient partials).  Calls that overlap on one workspace race.
 */
size_t nc_epilogue_workspace_size(int B, int M, int h, int w);

/*
 * pallas_fused_roi_step_epilogue forward (kernels_pallas.py:663-866):
 *   zhat = standardize(z + (has_border ? delta : 0)) per (b, m) plane (two-pass population
 *   variance, eps 1e-5); out = w_eff * sum_m zhat + s_eff * sum_m act(zhat + b_roi).
 * z (B,M,h,w), delta (M,h,w), w_eff/s_eff/b_roi (h,w) -> out (B,h,w), mean/rstd (B,M).
 * N = h*w <= 8192 runs a single pass per sample; larger planes run the tiled (B,M,tiles)
 * Chan parallel-variance pipeline.
 */
int nc_epilogue_fwd(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                    int has_border, const float* z, const float* delta, const float* w_eff,
                    const float* s_eff, const float* b_roi, float* out, float* mean, float* rstd,
                    void* ws, size_t ws_bytes);

/*
 * The number G >= 1 of partial output planes per sample that nc_epilogue_fwd_parts writes at
 * these shapes (its workgroups split the directions into G groups at small batches).
 */
int nc_epilogue_fwd_partials(int B, int M, int h, int w);

/*
 * nc_epilogue_fwd leaving the direction groups' partial outputs uncombined: parts (G, B, h, w)
 * with G = nc_epilogue_fwd_partials(B, M, h, w), whose sum over g in increasing order is out
 * (bit for bit).  nc_fftconv_fwd_parts consumes them directly, so the combine costs no launch.
 * No counterpart in the reference (whose epilogue is one fused op).
 */
int nc_epilogue_fwd_parts(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                          int has_border, const float* z, const float* delta, const float* w_eff,
                          const float* s_eff, const float* b_roi, float* parts, float* mean,
                          float* rstd, void* ws, size_t ws_bytes);

/*
 * The cell spectra of one propagation step: xhat (B, fft_h, fft_w/2+1) complex = rfft2 of
 * the cell state x = sum over q < n_parts of x_parts[q] (n_parts, B, hin, win), summed in
 * increasing q, plus xhat_add (one (fft_h, fft_w/2+1) spectrum, or NULL) - the first half of
 * nc_fftconv_fwd_parts (kernels_pallas.py:1779-1791).  No counterpart in the reference.
 */
int nc_fftconv_spectra(void* stream, int B, int hin, int win, int fft_h, int fft_w,
                       const float* x_parts, int n_parts, const float* xhat_add, float* xhat);

/*
 * The number G >= 1 of partial output planes per sample that nc_fftconv_epilogue_fwd writes:
 * ceil(M/4) where the fused kernel runs (the 64-wide grids, planes whose staging fits), else
 * nc_epilogue_fwd_partials(B, M, h, w).
 */
int nc_fftconv_epilogue_partials(int B, int M, int h, int w, int fft_h, int fft_w);

/*
 * The correlation step (nc_spectral_correlate) and the hidden-step epilogue without a border
 * term (nc_epilogue_fwd_parts with has_border = 0) as one operation - kernels_pallas.py:
 * 1779-1791 followed by 163-291: parts (G, B, hout, wout) with G =
 * nc_fftconv_epilogue_partials, mean/rstd (B, M).  z (B, M, hout, wout) receives the
 * correlation when not NULL (a training forward keeps it for the backward); on the 64-wide
 * grids it may be NULL (evaluation), elsewhere it is required as the epilogue's input.  ws:
 * nc_epilogue_workspace_size(B, M, hout, wout) bytes where the fused kernel does not run
 * (unused, may be NULL, where it does); on the 128- and 256-point grids a ws of at least
 * nc_fftconv_correlate_workspace_size bytes as well lets the correlation run as two
 * transform passes through it.  No counterpart in the reference (two ops there).
 */
int nc_fftconv_epilogue_fwd(void* stream, int B, int M, int hout, int wout, int pad_h,
                            int pad_w, int fft_h, int fft_w, const float* xhat,
                            const float* ghat, int act, float neg_slope, const float* w_eff,
                            const float* s_eff, const float* b_roi, float* z, float* parts,
                            float* mean, float* rstd, void* ws, size_t ws_bytes);

/*
 * Workspace bytes that let nc_fftconv_epilogue_fwd and nc_fftconv_port_fwd run a large-grid
 * correlation (an axis of 128 or 256 points) as two transform passes - a column pass over
 * the B*M products xhat_b * ghat_m, then a row pass, B*M*hout*fft_w/2 complex values in
 * between - instead of one workgroup per plane segment; 0 on the other grids.  The same
 * results to rounding (the passes and their bin order are the same).  It also holds the
 * per-band plane statistics with which nc_fftconv_epilogue_fwd's row pass hands the tiled
 * epilogue (hout*wout > 8192) its mean and variance, so that epilogue reads z once instead
 * of twice.  No counterpart in the reference.
 */
size_t nc_fftconv_correlate_workspace_size(int B, int M, int hout, int wout, int fft_h,
                                           int fft_w);

/*
 * Workspace bytes for nc_fftconv_port_fwd: nc_epilogue_workspace_size, or the fused kernel's
 * direction-group partial sums (2 * ceil(M/4) * B * n_port floats) where that is larger.
 * (nc_fftconv_correlate_workspace_size on top enables the two-pass large-grid correlation.)
 */
size_t nc_fftconv_port_workspace_size(int B, int M, int h, int w, int fft_h, int fft_w,
                                      int n_port);

/*
 * The last step's correlation (nc_spectral_correlate) and the output-port epilogue without a
 * border term (nc_port_fwd with has_border = 0) as one operation - kernels_pallas.py:1779-1791
 * followed by 1284-1347 and 1510-1551: out (B, P), zo (B, M, P), mean/rstd (B, M), pre (B, P)
 * as nc_port_fwd.  z (B, M, hout, wout) receives the correlation when not NULL (a training
 * forward keeps it for the backward); on the 32x64 and 64x64 grids it may be NULL
 * (evaluation: the planes are standardised on chip and only the port cells leave it),
 * elsewhere it is required.  n_port <= 256.  No counterpart in the reference (two ops there).
 */
int nc_fftconv_port_fwd(void* stream, int B, int M, int hout, int wout, int pad_h, int pad_w,
                        int fft_h, int fft_w, const float* xhat, const float* ghat,
                        int final_act, float neg_slope, int n_port, const int32_t* port_idx,
                        const float* port_params, float* z, float* out, float* zo, float* mean,
                        float* rstd, float* pre, void* ws, size_t ws_bytes);

/*
 * The output port when it covers the whole (sub-)ROI in row-major order (P = h*w: the Game of
 * Life chip's universe port, topology.py:359-388).  pallas_fused_output_port_epilogue
 * (kernels_pallas.py:1510-1551) for such a port is the hidden epilogue with the port
 * parameters (w_eff_out, s_eff_out, b_out) and the final activation in its place
 * (nc_fftconv_epilogue_fwd or nc_epilogue_fwd_parts with act = final_act), finished here:
 * out (n = B*P) = final_act(sum over g < G of parts[g]), pre (n) = that sum (may be NULL when
 * final_act is identity: port_out's identity form is the same sum).  Its reverse
 * nc_port_dense_bwd gives g_pre = g_out * final_act'(pre), the gy of nc_epilogue_bwd_parts.
 * No counterpart in the reference (whose port kernels gather P cells).
 */
int nc_port_dense_fwd(void* stream, int n, int G, int final_act, float neg_slope,
                      const float* parts, float* out, float* pre);
int nc_port_dense_bwd(void* stream, int n, int final_act, float neg_slope, const float* pre,
                      const float* g_out, float* g_pre);

/*
 * standardize_spatial_nchw (epilogue.py:20-25, jax.nn.standardize over the plane axes):
 * out = (x - mean) * rstd per plane, nplanes planes of n contiguous floats, with two-pass
 * population statistics and rstd = 1/sqrt(var + 1e-5) saved (nplanes each).  The reverse:
 * gx = rstd * (g - mean(g) - zhat * mean(g * zhat)), zhat recomputed from x, mean, rstd.
 */
int nc_standardize_fwd(void* stream, int nplanes, int n, const float* x, float* out,
                       float* mean, float* rstd);
int nc_standardize_bwd(void* stream, int nplanes, int n, const float* x, const float* mean,
                       const float* rstd, const float* g, float* gx);

/*
 * pallas_fused_roi_step_epilogue backward rule (kernels_pallas.py:869-1064): writes gz
 * (B,M,h,w), gdb = sum_b gz (M,h,w) when has_border, exact zeros without the border term
 * (kernels_pallas.py:1060), when gdb is not NULL (a caller that forms the border
 * cotangent from the spectra, nc_fftconv_bwd_ex, passes NULL) and gw/gs/gb (h,w).
 * gw/gs/gb are overwritten, or added to when accumulate_params; gdb is overwritten, or added
 * to when accumulate_gdb (a d-step reverse pass sums both over steps).
 */
int nc_epilogue_bwd(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                    int has_border, const float* z, const float* delta, const float* w_eff,
                    const float* s_eff, const float* b_roi, const float* mean, const float* rstd,
                    const float* gy, float* gz, float* gdb, float* gw, float* gs, float* gb,
                    int accumulate_params, int accumulate_gdb, void* ws, size_t ws_bytes);

/*
 * nc_epilogue_bwd without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  No counterpart in the reference.  Same arguments (minus ws, ws_bytes) and
 * results as nc_epilogue_bwd; its scratch is a file-scope device array of
 * NC_NOALLOC_SCRATCH_BYTES per GPU (16 MiB: the 40x50 ROI at B = 128 needs 11.7 MB, the
 * 24x32 crop at B = 512 9.0 MB, the 112x112 ROI at B = 64 13.4 MB), so shapes whose
 * nc_epilogue_workspace_size exceeds it (e.g. 224x224 at B = 32, M = 32: 26.7 MB) return
 * NC_ERR_SCRATCH_LIMIT.  Runs on the current device; a non-NULL stream must belong to it
 * (NC_ERR_INVALID_ARGUMENT otherwise).  Calls no allocator.  All calls on one GPU share its
 * scratch: calls that overlap on one GPU (concurrent streams or host threads) race.
 */
int nc_epilogue_bwd_noalloc(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                            int has_border, const float* z, const float* delta,
                            const float* w_eff, const float* s_eff, const float* b_roi,
                            const float* mean, const float* rstd, const float* gy, float* gz,
                            float* gdb, float* gw, float* gs, float* gb, int accumulate_params,
                            int accumulate_gdb);

/* The partial rows per parameter plane nc_epilogue_bwd_parts writes at these shapes. */
int nc_epilogue_bwd_partials(int B, int M, int h, int w);

/*
 * nc_epilogue_bwd leaving the parameter gradients as partial rows: gw rows at pg_rows, gs rows
 * at pg_rows + plane_stride, gb rows at pg_rows + 2*plane_stride (each R x (h*w) floats,
 * R = nc_epilogue_bwd_partials(B, M, h, w), plane_stride >= R*h*w); their row sums are
 * gw / gs / gb.  A d-step reverse pass gives each step its own R rows of one stack and sums
 * them all with one nc_rows_sum.  No border cotangent.  No counterpart in the reference.
 */
int nc_epilogue_bwd_parts(void* stream, int B, int M, int h, int w, int act, float neg_slope,
                          int has_border, const float* z, const float* delta, const float* w_eff,
                          const float* s_eff, const float* b_roi, const float* mean,
                          const float* rstd, const float* gy, float* gz, float* pg_rows,
                          size_t plane_stride, void* ws, size_t ws_bytes);

/*
 * pallas_standardize_output_port + pallas_fused_output_port_epilogue forward
 * (kernels_pallas.py:1256-1347, 1510-1551): per-plane (mean, rstd) over the whole (h,w)
 * plane, standardisation of the P port cells only (port_idx (P) int32 flat indices into the
 * (h,w) plane, in port order), then the port Codd algebra.  port_params (3,P) =
 * [w_eff_out, s_eff_out, b_out].  Writes out (B,P), zo (B,M,P), mean/rstd (B,M) and, when
 * final_act != identity, pre (B,P) (the pre-activation residual).  ws: nc_epilogue_workspace_size
 * bytes (planes above 8192 pixels use it for the tiled Chan statistics, smaller batches for the
 * split over directions).
 * port_params == NULL is pallas_standardize_output_port alone (kernels_pallas.py:1284-1347):
 * only zo, mean and rstd are written; out, pre and final_act are ignored.
 */
int nc_port_fwd(void* stream, int B, int M, int h, int w, int has_border, int final_act,
                float neg_slope, int n_port, const int32_t* port_idx, const float* z,
                const float* delta, const float* port_params, float* out, float* zo,
                float* mean, float* rstd, float* pre, void* ws, size_t ws_bytes);

/*
 * Backward of nc_port_fwd (kernels_pallas.py:1350-1504, 1538-1551): dense
 * gz = -rstd*(c1 + zhat*c2) plus rstd*g scattered at the port cells in registers; gdb =
 * sum_b gz when has_border (exact zeros without it) and gdb is not NULL; gdb and
 * g_port_params (3,P) overwritten, or
 * added to when accumulate_params.  With port_params == NULL (standardisation only, kernels_pallas.py:
 * 1350-1504) g_out is the (B,M,P) cotangent of zo and g_port_params is not touched.
 */
int nc_port_bwd(void* stream, int B, int M, int h, int w, int has_border, int final_act,
                float neg_slope, int n_port, const int32_t* port_idx, const float* z,
                const float* delta, const float* port_params, const float* zo,
                const float* mean, const float* rstd, const float* pre, const float* g_out,
                float* gz, float* gdb, float* g_port_params, int accumulate_params, void* ws,
                size_t ws_bytes);

/*
 * nc_port_bwd leaving the port-parameter gradients as partial rows: B rows of n_port floats
 * for each of the three parameters, planes plane_stride (>= B*n_port) floats apart from
 * pp_rows; their row sums are g_port_params.  Requires port_params; no border cotangent.
 * No counterpart in the reference.
 */
int nc_port_bwd_parts(void* stream, int B, int M, int h, int w, int has_border, int final_act,
                      float neg_slope, int n_port, const int32_t* port_idx, const float* z,
                      const float* delta, const float* port_params, const float* zo,
                      const float* mean, const float* rstd, const float* pre,
                      const float* g_out, float* gz, float* pp_rows, size_t plane_stride,
                      void* ws, size_t ws_bytes);

/* One job of nc_rows_sum: out[x] (+)= sum over r < nrows of rows[r*len + x], x < len. */
typedef struct nc_rows_job {
    const float* rows;
    float* out;
    int len;
    int accumulate;
    int nrows;
} nc_rows_job;

/*
 * Up to 10 row-stack sums in one launch, each in a fixed order (deterministic): the partial
 * rows of nc_fftconv_bwd_parts (complex spectra as float pairs), nc_epilogue_bwd_parts and
 * nc_port_bwd_parts, gathered over a reverse pass.  No counterpart in the reference.
 */
int nc_rows_sum(void* stream, int n_jobs, const nc_rows_job* jobs);

/* ---------------- piece 4: adaptive active-region bucketing ---------------------------- */

/*
 * _compute_adaptive_mask_tensors (adaptive_mask.py:200-315) over the full ROI: writes
 * stats[8] = {r_eff_h, r_eff_w, salient_count, any_active, r0, r1, c0, c1} and the dilated
 * active mask (roi_h, roi_w) u8.  act_roi (roi_h, roi_w) may be NULL.  The bucket
 * quantisation (adaptive_mask.py:105-161) is host integer logic on these 8 values.
 */
int nc_adaptive_stats(void* stream, const nc_chip_desc* chip, const float* cell,
                      const float* filters, const uint8_t* io_mask_roi, const float* act_roi,
                      int margin_h, int margin_w, float salience_threshold, float bias_threshold,
                      float filter_threshold, float activity_threshold, int32_t* stats,
                      uint8_t* dilated);

/* ---------------- orchestration helpers ------------------------------------------------- */

/*
 * inject_inputs_roi_2d (propagator.py:135-191) as a gather: roi[b, i] = inputs[b, src[i]]
 * when src[i] >= 0, else 0, for the n_roi cells of the (cropped) ROI.  The host builds src
 * from the port geometry once (later ports win on overlap, as the reference's sequential
 * .at[].set does).
 */
int nc_inject_roi(void* stream, int B, int n_in, const float* inputs, int n_roi,
                  const int32_t* src, float* roi);

/* default_mse_loss (trainer.py:57-61): loss[0] = mean((pred-target)^2); g_pred = 2(pred-target)/n. */
int nc_mse_loss(void* stream, int n, const float* pred, const float* target, float* loss,
                float* g_pred);

/*
 * One batch of VNNTrainer.evaluate_packed (trainer.py:49-54, 122-138): for each sample b the 8
 * port outputs out[b, 0..7] are rounded half-to-even, saturated to uint8 (NaN -> 0) and packed
 * MSB-first (BIT_WEIGHTS_U8, trainer.py:20) into preds_packed[b] (may be NULL); then
 * acc[0] += mean_b(preds_packed[b] == y_packed[b]) in fp32.  n_out must be 8.
 */
int nc_packed_accuracy(void* stream, int B, int n_out, const float* out,
                       const uint8_t* y_packed, uint8_t* preds_packed, float* acc);

/*
 * optax.adamw(learning_rate) update as applied by VNNTrainer (trainer.py:101-106): with
 * c = count[0] (the number of earlier updates), m,v moments, bias correction by c+1, and
 * p -= lr[min(c, n_lr-1)] * (mhat/(sqrt(vhat)+eps) + weight_decay * p); then count[0] = c+1.
 * ``lr`` is a device table of the learning-rate schedule evaluated at 0..n_lr-1 (n_lr = 1 for a
 * constant rate; later steps reuse the last entry), so a captured graph replays the schedule.
 */
int nc_adamw_step(void* stream, int n, float* p, const float* g, float* m, float* v,
                  int32_t* count, const float* lr, int n_lr, float b1, float b2, float eps,
                  float weight_decay);

#ifdef __cplusplus
}
#endif

#endif /* NEUROCELL_HIP_H_ */

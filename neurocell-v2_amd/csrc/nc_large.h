// Internal interface between the C ABI entry points (nc_spectral.hip) and the large-grid
// spectral kernels (nc_spectral_large.hip): FFT grids with an axis of 128 or 256 points and
// both axes in {64, 128, 256}.  Arguments have the meaning of the matching nc_* entry points.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

bool nc_large_grid(int fft_h, int fft_w);

int nc_large_filter_spectrum_fwd(hipStream_t st, int M, int kh, int kw, int fft_h, int fft_w,
                                 const float* filters, float* ghat);

int nc_large_filter_spectrum_bwd(hipStream_t st, int M, int kh, int kw, int fft_h, int fft_w,
                                 int shift_h, int shift_w, const float* dghat, float* g_filters,
                                 int accumulate, int conj_in);

int nc_large_fftconv_fwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout,
                         int pad_h, int pad_w, int fft_h, int fft_w, const float* x, int n_parts,
                         const float* xhat_add, const float* ghat, float* z, float* xhat);

int nc_large_plane_spectrum(hipStream_t st, int nplanes, int hin, int win, int fft_h, int fft_w,
                            int shift_h, int shift_w, const float* x, float* xhat);

struct nc_spectrum_job;
int nc_large_plane_spectra(hipStream_t st, int fft_h, int fft_w, int n_jobs,
                           const nc_spectrum_job* jobs);

// The segmented (workgroup-per-plane) transforms on the 64 x 64 grid as well as the large ones,
// for per-sample jobs where the wavefront-per-plane kernels leave most of the chip idle:
// half-spectra of nplanes planes (each the sum of nparts partial planes qstride floats apart;
// flip / add / shift as nc_spectrum_job) and the dx inverse of B unpacked dx spectra, each
// the sum of nchunk partials (nchunk, B, F).
int nc_seg_rfft2(hipStream_t st, int fft_h, int fft_w, int nplanes, int hin, int win, int flip,
                 const float* x, void* xhat, const void* add, int shift_h, int shift_w,
                 int nparts, size_t qstride);
int nc_seg_dx(hipStream_t st, int B, int nchunk, int hin, int win, int pad_h, int pad_w,
              int fft_h, int fft_w, const void* dx_spectra, float* dx);

// z = the correlation's window of irfft2(xhat_b * ghat_m); with a workspace of at least
// nc_large_correlate_ws bytes, by the two-pass transform (column pass, then row pass, the
// intermediate in ws), else one workgroup per plane segment.  band_stats (two-pass only,
// else NC_ERR_UNSUPPORTED): the row pass also writes each plane's band statistics, layout
// (2, B*M, ceil(hout / nc_large_band_rows)) of (sum, centred sum of squares), a band being
// nc_large_band_rows consecutive output rows; the workspace keeps them at
// nc_large_band_stats_offset bytes, past the intermediate.
int nc_large_correlate(hipStream_t st, int B, int M, int hout, int wout, int pad_h, int pad_w,
                       int fft_h, int fft_w, const float* xhat, const float* ghat, float* z,
                       void* ws = nullptr, size_t ws_bytes = 0, float* band_stats = nullptr);
size_t nc_large_correlate_ws(int B, int M, int hout, int fft_h, int fft_w);
int nc_large_band_rows(int fft_h, int fft_w);
size_t nc_large_band_stats_offset(int B, int M, int hout, int fft_h, int fft_w);

// Implemented in nc_epilogue.hip: whether an (n_pix)-pixel plane takes the tiled epilogue,
// and its forward from given tile statistics (2, B*M, T) of tiles of tile_pix consecutive
// pixels (the last one partial), without a border term: out (B, N), mean / rstd (B, M).
bool nc_epilogue_tiled(int n_pix);
// The tiled epilogue backward's first stage alone (no border term), for a caller that forms
// gz itself: the gw / gs / gb partial rows into pg_rows (nc_epilogue_bwd_parts' layout) and
// the per-tile (c1, c2) partials, layout (2, B, M, *n_tiles), at *cpart inside ws.
int nc_epilogue_bwd_stage1(hipStream_t st, int B, int M, int h, int w, int act, float neg_slope,
                           const float* z, const float* w_eff, const float* s_eff,
                           const float* b_roi, const float* mean, const float* rstd,
                           const float* gy, float* pg_rows, size_t plane_stride, void* ws,
                           size_t ws_bytes, const float** cpart, int* n_tiles);

// gz of the tiled epilogue backward, formed where it is read (the arithmetic of its second
// stage): gz = rstd * (gy * (w + s * act'(zhat + b)) - c1 - zhat * c2), zhat = (z - mean) *
// rstd, (c1, c2) = the plane's tile partials summed over its n_tiles tiles, divided by h*w.
struct nc_epi_gz {
    const float *z, *w_eff, *s_eff, *b_roi, *gy, *mean, *rstd, *cpart;
    int n_tiles, act;
    float neg_slope;
};
// nc_large_fftconv_bwd with its cotangent planes gz given that way (hout x wout planes).
int nc_large_fftconv_bwd_epi(hipStream_t st, int B, int M, int hin, int win, int hout,
                             int wout, int pad_h, int pad_w, int fft_h, int fft_w,
                             const nc_epi_gz& gz, const float* xhat, const float* ghat,
                             int need_dx, float* dx, float* dghat, int accumulate,
                             int conj_dghat, float* gz_hat_sum, int sum_accumulate, int parts,
                             void* ws);
int nc_epilogue_fwd_from_stats(hipStream_t st, int B, int M, int h, int w, int act,
                               float neg_slope, const float* z, const float* w_eff,
                               const float* s_eff, const float* b_roi, const float* stats,
                               int n_tiles, int tile_pix, float* out, float* mean, float* rstd);

size_t nc_large_fftconv_bwd_ws(int B, int M, int fft_h, int fft_w);

// parts: dghat / gz_hat_sum are nc_large_red_splits(...) row stacks (one row per sample
// slice of the reduction, each accumulated into when accumulate / sum_accumulate), else
// single sums.
int nc_large_fftconv_bwd(hipStream_t st, int B, int M, int hin, int win, int hout, int wout,
                         int pad_h, int pad_w, int fft_h, int fft_w, const float* gz,
                         const float* xhat, const float* ghat, int need_dx, float* dx,
                         float* dghat, int accumulate, int conj_dghat, float* gz_hat_sum,
                         int sum_accumulate, int parts, void* ws);
int nc_large_red_splits(int B, int M, int fft_h, int fft_w);

// dx = the inverse of one sample's unpacked dx half-spectrum with the unshifted roll.
int nc_large_hat_dx(hipStream_t st, int hin, int win, int pad_h, int pad_w, int fft_h, int fft_w,
                    const void* dx_spectrum, float* dx);

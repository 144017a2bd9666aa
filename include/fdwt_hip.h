/*
 * fdwt_hip.h -- C ABI of the MI355X (gfx950) HIP kernels behind pytorch_morlet_fdwt_amd.
 *
 * Every entry point takes raw device pointers, int64 sizes, small int parameters and the
 * hipStream_t to launch on (passed as void*).  None of them allocates memory or
 * synchronises the host; all work is enqueued on `stream`.  Return value: 0 on success, a
 * positive hipError_t code if a launch failed, or a negative FDWT_ERR_* code if the
 * arguments were rejected before anything was launched (see fdwt_error_string).
 *
 * Each entry point replaces one launcher of the reference package
 * (pytorch_morlet_fdwt, src/fdwt/kernels/); the citation is given per function.
 * Rows are contiguous: element (r, i) of an (R, N) signal is at r * N + i.
 */
#ifndef FDWT_HIP_H_
#define FDWT_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* storage dtypes of signals / coefficients.  F32, F16 and BF16 compute in fp32 (filters
 * are passed as fp32), F64 computes in fp64 (filters passed as fp64). */
#define FDWT_F32 0
#define FDWT_F64 1
#define FDWT_F16 2
#define FDWT_BF16 3
/* fp32 storage with bf16 matrix-core operands and fp32 accumulation (the reference's "bf16"
 * precision, conv.py:332-338): accepted by fdwt_morlet_backward_x (matrix-core adjoint) and
 * fdwt_morlet_backward_h (matrix-core filter gradient); stages that run on the vector kernels
 * compute in fp32 */
#define FDWT_F32_BF16 4

/* boundary modes, numbered as the reference's MODES table (kernels/dwt.py:30) */
#define FDWT_MODE_ZERO 0
#define FDWT_MODE_PERIODIC 1
#define FDWT_MODE_SYMMETRIC 2
#define FDWT_MODE_REFLECT 3
#define FDWT_MODE_PERIODIZATION 4

#define FDWT_ERR_ARG (-1)         /* invalid size / mode / dtype / null pointer */
#define FDWT_ERR_TOO_LONG (-2)    /* a row does not fit the kernel's on-chip buffers */
#define FDWT_ERR_SCRATCH (-3)    /* a call needs more than the fixed scratch of a no-allocation entry */
#define FDWT_MAX_LEVELS 32
#define FDWT_SYN_MAX_LEVELS 16   /* levels per fdwt_synthesis_chain call */

/* Error message for a return code of this library (or a hipError_t). */
const char* fdwt_error_string(int code);

/* Library build tag, e.g. "fdwt-hip gfx950". */
const char* fdwt_version(void);

/* ---------------------------------------------------------------- DWT, one level
 *
 * fdwt_dwt_analysis -- replaces `analysis(x, h0, h1, mode, off, n_out)`
 * (src/fdwt/kernels/dwt.py:191-206):
 *     y_b[r, o] = sum_{j<taps} h_b[j] * x_ext[r, 2*o + off - j],   b = 0, 1
 * x: (rows, n) -> y0, y1: (rows, n_out), all of storage dtype `dtype`; h0, h1: `taps`
 * filter coefficients (fp32, or fp64 for FDWT_F64).  `taps` must be even.
 */
int fdwt_dwt_analysis(const void* x, void* y0, void* y1, const void* h0, const void* h1,
                      int64_t rows, int64_t n, int64_t n_out, int32_t taps, int32_t mode,
                      int32_t off, int32_t dtype, void* stream);

/* fdwt_dwt_synthesis -- replaces `synthesis(a, d, h0, h1, mode, off, n)`
 * (src/fdwt/kernels/dwt.py:209-228): the exact transpose of fdwt_dwt_analysis,
 *     y = A^T (a, d),  a, d: (rows, nc) -> y: (rows, n).
 * `a` or `d` may be NULL (read as zeros). */
int fdwt_dwt_synthesis(const void* a, const void* d, void* y, const void* h0, const void* h1,
                       int64_t rows, int64_t nc, int64_t n, int32_t taps, int32_t mode,
                       int32_t off, int32_t dtype, void* stream);

/* ---------------------------------------------------------------- DWT, fused levels
 *
 * fdwt_analysis_chain -- `levels` analysis levels in one launch, replacing the per-level
 * loops of wavedec (src/fdwt/dwt.py:146-158) and of the backward of waverec
 * (dwt.py:161-171 with _Synthesis.backward, dwt.py:75-82).  Level l (0-based) analyses a
 * signal of length n_in[l] into two bands of length n_out[l]; the input of level 0 is x,
 * the input of level l > 0 is the low band of level l - 1 followed by
 * n_in[l] - n_out[l - 1] (0 or 1) zeros.  details[l] receives the high band of level l,
 * approx the low band of the last level.  Each row stays on chip across levels, so x is
 * read once and every band is written once.
 */
int fdwt_analysis_chain(const void* x, void* const* details, void* approx, const void* h0,
                        const void* h1, int64_t rows, const int64_t* n_in,
                        const int64_t* n_out, int32_t levels, int32_t taps, int32_t mode,
                        int32_t off, int32_t dtype, void* stream);

/* fdwt_synthesis_chain -- the transpose direction: `levels` synthesis levels in one
 * launch, replacing the per-level loop of waverec (dwt.py:161-171) and of the backward of
 * wavedec.  Level l (0-based, coarsest first) combines a low band of length nc[l] with
 * details[l] (length nc[l]; NULL = zeros) into a signal of length n_out[l].  The low band
 * of level 0 is approx (NULL = zeros); the low band of level l > 0 is the first nc[l]
 * samples of the output of level l - 1 (nc[l] is n_out[l-1] or n_out[l-1] - 1, the
 * pywt.waverec trim).  out receives the output of the last level.  At most
 * FDWT_SYN_MAX_LEVELS levels per call (longer chains run as consecutive calls).
 */
int fdwt_synthesis_chain(const void* approx, const void* const* details, void* out,
                         const void* h0, const void* h1, int64_t rows, const int64_t* nc,
                         const int64_t* n_out, int32_t levels, int32_t taps, int32_t mode,
                         int32_t off, int32_t dtype, void* stream);

/* Largest row length (in samples) that the fused chain kernels keep on chip for a given
 * filter length and dtype; longer rows must first be reduced with fdwt_dwt_analysis. */
int64_t fdwt_chain_max_length(int32_t taps, int32_t dtype);

/* ---------------------------------------------------------------- Morlet CWT pyramid
 *
 * One octave ("stage") of the pyramid convolves a chain signal x_j (rows, n_in) with
 * n_scales Morlet filters dilated by dil = 2^j:
 *     W_s[r, n] = sum_{t=-half}^{half} H_s[c + t] * x_j[r, n + x_off - dil * t]
 * Filters are given as a tap table taps[s][t][ch] = H_{s,ch}[c + t], t = 0..half, ch = re
 * (and im when channels == 2); real parts must be even and imaginary parts odd around c, as
 * every Morlet filter is.  support[s] (non-decreasing) bounds the non-zero taps of scale s,
 * chan[s] is its output channel.  support / chan are host arrays of n_scales entries
 * (n_scales <= FDWT_CWT_MAX_SCALES).  Compute dtypes: FDWT_F32 or FDWT_F64.  Calls with
 * rows == 0 or n_out == 0 do nothing; otherwise the stage entry points that read x
 * (forward, backward_h, mix, softmax) need n_in >= 1 and return FDWT_ERR_ARG for n_in == 0.
 */
#define FDWT_CWT_MAX_SCALES 64

/* Sampled Morlet filter bank, replacing `MorletPlan.filters(scales, w0, dtype)`
 * (src/fdwt/cwt.py:181-203) on the device: H (n_scales * channels, 2 center + 1) in dtype,
 * row i * channels + ch, column center + k, for scale scales[i] sampled at spacing dil[i]
 * and truncated to |k| <= support[i]; channels 2 = re / im rows, 1 = real only; norm_l2 = 1
 * for the 1/sqrt(s) normalisation, 0 for 1/s.  scales (n_scales) and w0 (1) are float64
 * device arrays, dil / support host arrays (n_scales <= FDWT_MORLET_MAX_FILTERS).  Values are
 * computed in float64 at |k| and mirrored, so rows are exactly even (re) / odd (im). */
#define FDWT_MORLET_MAX_FILTERS 256
int fdwt_morlet_filters(const double* scales, const double* w0, const int32_t* dil,
                        const int32_t* support, int32_t n_scales, int32_t center,
                        int32_t channels, int32_t norm_l2, void* H, int32_t dtype, void* stream);

/* Gradient of fdwt_morlet_filters, replacing autograd through the torch construction of
 * cwt.py:181-203: writes g_scales[i] = sum_k gH[i, k] dH[i, k]/ds_i and
 * g_w0[0] = sum gH dH/dw0 (float64 device arrays; gH in dtype, the shape of H).  One
 * workgroup, fixed summation order (deterministic). */
int fdwt_morlet_filters_backward(const double* scales, const double* w0, const int32_t* dil,
                                 const int32_t* support, int32_t n_scales, int32_t center,
                                 int32_t channels, int32_t norm_l2, const void* gH,
                                 int32_t dtype, double* g_scales, double* g_w0, void* stream);

/* replaces the half-band launcher `halfband(x, taps, y, off, dil, transpose, accumulate)`
 * (src/fdwt/kernels/conv.py:411-430):
 *   y[r, n] (+)= taps[0] x[r, n + b] + sum_{t odd <= c} taps[t] (x[r, n + b - dil t] + x[r, n + b + dil t])
 * with b = off - dil * c (forward) or dil * c - off (transpose); x is zero outside [0, n_in). */
int fdwt_halfband(const void* x, const void* taps, void* y, int64_t rows, int64_t n_in,
                  int64_t n_out, int32_t c, int64_t b, int32_t dil, int32_t accumulate,
                  int32_t dtype, void* stream);

/* replaces `forward(x, hT, kb, cmap, y, off, dil, block_s)` (conv.py:306-329): writes
 * y[r, chan[s], n, ch] (y: (rows, s_total, n_out, channels), interleaved re / im). */
int fdwt_morlet_forward(const void* x, const void* taps, void* y, int64_t rows, int64_t n_in,
                        int64_t n_out, int64_t x_off, int32_t n_scales, int32_t half,
                        const int32_t* support, const int32_t* chan, int32_t dil,
                        int32_t channels, int32_t s_total, int32_t dtype, void* stream);

/* replaces `backward_x(g, h, kf, cmap, gx, off, dil, accumulate)` (conv.py:345-369): the
 * adjoint of fdwt_morlet_forward, gx (rows, n_in) (+)= A^T g with g (rows, g_scales, n_out,
 * channels) read at channels chan[s]. */
int fdwt_morlet_backward_x(const void* g, const void* taps, void* gx, int64_t rows,
                           int64_t n_in, int64_t n_out, int64_t x_off, int32_t n_scales,
                           int32_t half, const int32_t* support, const int32_t* chan,
                           int32_t dil, int32_t channels, int32_t g_scales, int32_t accumulate,
                           int32_t dtype, void* stream);

/* replaces `backward_h(x, g, kb, cmap, off, dil, K, block_s)` (conv.py:372-408): gradient of
 * every tap, gh[s][k][ch] (+)= sum_{r,n} g[r, chan[s], n, ch] x[r, n + x_off - dil (k - half)],
 * k = 0..2 half; gh: (n_scales, 2 half + 1, channels).  Deterministic: per-workgroup partial
 * sums go to the caller's workspace (fdwt_morlet_backward_h_workspace elements), then one
 * fixed-order reduction. */
int64_t fdwt_morlet_backward_h_workspace(int64_t rows, int64_t n_out, int32_t n_scales,
                                         int32_t half, int32_t channels);
int fdwt_morlet_backward_h(const void* x, const void* g, void* workspace,
                           int64_t workspace_elems, void* gh, int64_t rows, int64_t n_in,
                           int64_t n_out, int64_t x_off, int32_t n_scales, int32_t half,
                           const int32_t* support, const int32_t* chan, int32_t dil,
                           int32_t channels, int32_t g_scales, int32_t accumulate,
                           int32_t dtype, void* stream);

/* No counterpart in the reference: fdwt_morlet_backward_h for callers that cannot allocate
 * (code under HIP graph capture, allocation-free serving loops).  Same arguments without the
 * workspace, same kernels and result bit for bit; the partial sums go to a fixed array of
 * fdwt_morlet_backward_h_noalloc_capacity() bytes (32 MiB) in device memory, one per GPU,
 * held until the process ends.  A call whose partial sums do not fit returns FDWT_ERR_SCRATCH
 * before any launch (the matrix-core path needs resident-workgroups x n_scales x K x channels
 * elements, the vector path, K > 128, rows x ceil(n_out / 512) x the same).  All calls on one
 * GPU share that array: calls that overlap on one GPU (several streams or threads) race. */
int64_t fdwt_morlet_backward_h_noalloc_capacity(void);
int fdwt_morlet_backward_h_noalloc(const void* x, const void* g, void* gh, int64_t rows,
                                   int64_t n_in, int64_t n_out, int64_t x_off,
                                   int32_t n_scales, int32_t half, const int32_t* support,
                                   const int32_t* chan, int32_t dil, int32_t channels,
                                   int32_t g_scales, int32_t accumulate, int32_t dtype,
                                   void* stream);

/* Fused scalogram mix, replacing `mix_forward` / `mix_backward` (src/fdwt/kernels/mix.py:74-108):
 *   forward   y[r, n] (+)= sum_s a[d, chan[s]] |W_s| + b[d, chan[s]] Re W_s,  d = (r + row0) % d_dim
 *   backward  gw[r, s, n, ch] = dL/dW_s for the stage (gw: (rows, n_scales, n_out, channels)),
 *             and per-(row, tile) partial sums (sum gy |W_s|, sum gy Re W_s) in the workspace,
 *             laid out (rows, tiles, n_scales, 2); fdwt_mix_workspace gives its size.
 * a, b: (d_dim, s_total) compute dtype.  The scalogram is never written to memory. */
int64_t fdwt_mix_workspace(int64_t rows, int64_t n_out, int32_t n_scales);
int fdwt_mix_forward(const void* x, const void* taps, const void* a, const void* b, void* y,
                     int64_t rows, int64_t n_in, int64_t n_out, int64_t x_off,
                     int32_t n_scales, int32_t half, const int32_t* support,
                     const int32_t* chan, int32_t dil, int32_t channels, int32_t s_total,
                     int32_t d_dim, int64_t row0, int32_t accumulate, int32_t dtype,
                     void* stream);
int fdwt_mix_backward(const void* x, const void* taps, const void* a, const void* b,
                      const void* gy, void* gw, void* workspace, int64_t workspace_elems,
                      int64_t rows, int64_t n_in, int64_t n_out, int64_t x_off,
                      int32_t n_scales, int32_t half, const int32_t* support,
                      const int32_t* chan, int32_t dil, int32_t channels, int32_t s_total,
                      int32_t d_dim, int64_t row0, int32_t dtype, void* stream);

/* Spectral softmax stage, replacing `forward_stage` / `backward_stage`
 * (src/fdwt/kernels/softmax.py:195-210).  a_f = |W_f| * inv_tau; V is per channel
 * ((nch, v_s_total), row r uses V[(r + row0) % nch]) or per position ((G, v_s_total, n_out),
 * row r uses V[(r + row0) / nch]).
 *   forward  folds the stage into the online softmax state (m, l, num), each (rows, n_out);
 *            first = no state yet; last = write num / l (the output) into num.
 *   backward p = exp(a - m) / l, gp = gy p, writes gw (rows, n_scales, n_out, 2) =
 *            gp (V - out) inv_tau W / |W| and dL/dV partials in the workspace: per channel
 *            (rows, tiles, n_scales) sums over positions, per position (rows, n_scales, n_out)
 *            (fdwt_softmax_workspace elements). */
int fdwt_softmax_forward(const void* x, const void* taps, const void* v, int32_t v_per_position,
                         int64_t v_s_total, int32_t nch, void* m, void* l, void* num,
                         int64_t rows, int64_t n_in, int64_t n_out, int64_t x_off,
                         int32_t n_scales, int32_t half, const int32_t* support,
                         const int32_t* chan, int32_t dil, double inv_tau, int32_t first,
                         int32_t last, int32_t dtype, void* stream);
int64_t fdwt_softmax_workspace(int64_t rows, int64_t n_out, int32_t n_scales,
                               int32_t v_per_position);
int fdwt_softmax_backward(const void* x, const void* taps, const void* v,
                          int32_t v_per_position, int64_t v_s_total, int32_t nch, int64_t row0,
                          const void* m, const void* l, const void* out, const void* gy,
                          void* gw, void* workspace, int64_t workspace_elems, int64_t rows,
                          int64_t n_in, int64_t n_out, int64_t x_off, int32_t n_scales,
                          int32_t half, const int32_t* support, const int32_t* chan,
                          int32_t dil, double inv_tau, int32_t dtype, void* stream);

/* dL/dV of the per-position spectral softmax (v_per_position = 1): the backward's workspace
 * partials part ((groups * nch) rows, n_scales, n_out), summed over each group's nch rows in
 * row order (deterministic), are added to gv[g0 + g, chan[s], n] (gv: (v_groups, v_s_total,
 * n_out)).  Replaces the atomic dL/dV accumulation of the reference's backward stage
 * (src/fdwt/kernels/softmax.py:121-127, :208) for that V layout. */
int fdwt_softmax_dv_reduce(const void* part, void* gv, int64_t groups, int32_t nch,
                           int32_t n_scales, const int32_t* chan, int64_t v_groups,
                           int64_t v_s_total, int64_t n_out, int64_t g0, int32_t dtype,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FDWT_HIP_H_ */

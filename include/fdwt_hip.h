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

/* boundary modes, numbered as the reference's MODES table (kernels/dwt.py:30) */
#define FDWT_MODE_ZERO 0
#define FDWT_MODE_PERIODIC 1
#define FDWT_MODE_SYMMETRIC 2
#define FDWT_MODE_REFLECT 3
#define FDWT_MODE_PERIODIZATION 4

#define FDWT_ERR_ARG (-1)         /* invalid size / mode / dtype / null pointer */
#define FDWT_ERR_TOO_LONG (-2)    /* a row does not fit the kernel's on-chip buffers */
#define FDWT_MAX_LEVELS 32

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
 * pywt.waverec trim).  out receives the output of the last level.
 */
int fdwt_synthesis_chain(const void* approx, const void* const* details, void* out,
                         const void* h0, const void* h1, int64_t rows, const int64_t* nc,
                         const int64_t* n_out, int32_t levels, int32_t taps, int32_t mode,
                         int32_t off, int32_t dtype, void* stream);

/* Largest row length (in samples) that the fused chain kernels keep on chip for a given
 * filter length and dtype; longer rows must first be reduced with fdwt_dwt_analysis. */
int64_t fdwt_chain_max_length(int32_t taps, int32_t dtype);

#ifdef __cplusplus
}
#endif

#endif /* FDWT_HIP_H_ */

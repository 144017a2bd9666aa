// Morlet CWT pyramid kernels for gfx950: half-band chain step, Morlet filter bank (forward,
// adjoint, filter gradient), and the fused scalogram consumers (mix, spectral softmax).
//
// One octave ("stage") of the pyramid convolves the chain signal x_j with S_j Morlet
// filters dilated by dil = 2^j (reference: src/fdwt/kernels/conv.py:38-134, cwt.py:213-244):
//     W_s[n] = sum_{t=-half}^{half} H_s[c + t] x_j[n + x_off - dil t]
// Morlet filters are even (real part) and odd (imaginary part) around their centre c
// (cwt.py:194-203), so with n0 = n + x_off
//     Re W_s[n] = h_s[0] x[n0] + sum_{t>=1} h_s[t] (x[n0 - dil t] + x[n0 + dil t])
//     Im W_s[n] =                sum_{t>=1} g_s[t] (x[n0 - dil t] - x[n0 + dil t])
// with taps h_s[t] = Re H_s[c + t], g_s[t] = Im H_s[c + t].  The sums and differences of a
// tap pair are formed once per position and shared by every scale of the stage, halving
// the multiplies of a direct convolution.  The taps are passed as a compact table
// taps[s][t][ch] (t = 0..half, ch = re / im).
//
// Design: a workgroup owns one row and a tile of TT output positions; the tile of x_j it
// needs (TT + 2 dil half samples) is staged in LDS by coalesced loads; thread i handles
// positions n0 + i + NT v (v < V), so LDS reads of neighbouring lanes are neighbouring
// words (no bank conflicts) and every output store is coalesced.  Scales are processed in
// groups of SG with 2 V SG accumulators in registers.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace fdwt {
namespace {

constexpr int NT = 256;
constexpr int V = 4;
constexpr int TT = NT * V;        // output positions per workgroup
constexpr int SG = 8;             // scales per register group
constexpr int MAXS = FDWT_CWT_MAX_SCALES;

struct Stage {
  const void* x;     // (rows, n_in) chain signal of the stage
  const void* taps;  // (n_scales, half + 1, C) compute dtype
  int64_t n_in, n_out, x_off;
  int32_t n_scales, half, dil, C;
  int32_t sup[MAXS];   // per-scale half support (taps t > sup[s] are zero)
  int32_t chan[MAXS];  // global scale index of each local scale
};

template <typename T>
__device__ inline T load_clamped(const T* __restrict__ p, int64_t i, int64_t n) {
  const T w = p[min(max(i, (int64_t)0), n - 1)];
  return (i >= 0 && i < n) ? w : T(0);
}

// Magnitude |W| = sqrt(q) and its reciprocal (0 for q = 0) of a complex value with q = |W|^2,
// and the exponential of the online softmax.  float32 uses the hardware instructions
// v_sqrt_f32 / v_rsq_f32 / v_exp_f32 (about 1 ulp each; the correctly rounded library calls
// cost several times the instructions, comparable to a short filter's taps per scale), with
// v_rsq_f32's input scaled out of the denormal range; float64 keeps the library functions.
template <typename T>
__device__ inline T hw_sqrt(T q) {
  return sqrt(q);
}
template <>
__device__ inline float hw_sqrt<float>(float q) {
  return __builtin_amdgcn_sqrtf(q);
}
template <typename T>
__device__ inline void mag_inv(T q, T& mag, T& inv) {
  mag = sqrt(q);
  inv = mag > T(0) ? T(1) / mag : T(0);
}
template <>
__device__ inline void mag_inv<float>(float q, float& mag, float& inv) {
  const bool tiny = q < 0x1p-100f;
  const float r = __builtin_amdgcn_rsqf(tiny ? q * 0x1p+64f : q);
  inv = q > 0.0f ? (tiny ? r * 0x1p+32f : r) : 0.0f;
  mag = q * inv;
}
// Online-softmax exponentials: float32 keeps its running maximum in base 2 (v_exp_f32 computes
// 2^x; |W| / tau is scaled by log2 e once), float64 in base e.  The state in memory is base e.
template <typename T>
struct SoftExp {
  static constexpr T kLog = T(1);
  static __device__ T ex(T x) { return exp(x); }
};
template <>
struct SoftExp<float> {
  static constexpr float kLog = 1.44269504088896341f;  // log2 e
  static __device__ float ex(float x) { return __builtin_amdgcn_exp2f(x); }
};

// Raw buffer access to one array of `bytes` < 2^31 bytes: a load takes a 32-bit byte offset
// (one VGPR instead of a 64-bit address) and returns 0 for any offset outside [0, bytes),
// negative offsets included (they are range-checked as unsigned).  The resource is built in
// scalar registers; 0x00020000 is the gfx9 descriptor word 3 (32-bit data format, no swizzle).
struct BufRsrc {
  __amdgpu_buffer_rsrc_t r;
};
__device__ inline BufRsrc make_rsrc(const void* base, int64_t bytes) {
  return {__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                            0x00020000)};
}
template <typename T>
__device__ inline T buf_load(BufRsrc b, int byte_off);
template <>
__device__ inline float buf_load<float>(BufRsrc b, int byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b.r, byte_off, 0, 0));
}
template <>
__device__ inline double buf_load<double>(BufRsrc b, int byte_off) {
  return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(b.r, byte_off, 0, 0));
}

// Stage x[row][p0 .. p0 + span) into X (zero outside [0, n); n >= 1).  Eight loads per thread
// are issued before any is written to LDS (unconditional, from clamped indices; the range mask
// is applied at the write): a load-then-write loop waits for each load in turn.
template <typename T>
__device__ inline void stage_row(T* X, const T* __restrict__ xrow, int64_t p0, int span,
                                 int64_t n) {
  constexpr int SB = 8;
  for (int k0 = 0; k0 < span; k0 += SB * NT) {
    T v[SB];
#pragma unroll
    for (int r = 0; r < SB; ++r)
      v[r] = xrow[min(max(p0 + k0 + r * NT + threadIdx.x, (int64_t)0), n - 1)];
#pragma unroll
    for (int r = 0; r < SB; ++r) {
      const int k = k0 + r * NT + threadIdx.x;
      const int64_t i = p0 + k;
      if (k < span) X[k] = (i >= 0 && i < n) ? v[r] : T(0);
    }
  }
}

// Copy elements [k_begin, k_end) with eight loads per thread in flight: load(k) must be an
// unconditional load that is valid for every k in the range (clamped indices), store(k, v)
// applies any mask.  (A load-then-store loop waits for each load in turn.)
template <typename T, typename LoadF, typename StoreF>
__device__ inline void batched_copy(int k_begin, int k_end, LoadF&& load, StoreF&& store) {
  constexpr int SB = 8;
  for (int k0 = k_begin; k0 < k_end; k0 += SB * NT) {
    T v[SB];
#pragma unroll
    for (int r = 0; r < SB; ++r) v[r] = load(min(k0 + r * NT + (int)threadIdx.x, k_end - 1));
#pragma unroll
    for (int r = 0; r < SB; ++r) {
      const int k = k0 + r * NT + (int)threadIdx.x;
      if (k < k_end) store(k, v[r]);
    }
  }
}

// Scalogram of positions tid + NT v of the tile for the scale group [s0, s0 + ns), from the
// staged tile X whose element ci + dil * half corresponds to tile position ci.
template <typename T, bool CPLX>
__device__ inline void bank_group(const T* __restrict__ X, const T* __restrict__ taps, int half,
                                  int dil, int s0, int ns, int tmax, T (&re)[V][SG],
                                  T (&im)[V][SG]) {
  constexpr int C = CPLX ? 2 : 1;
  const int tid = threadIdx.x;
  const int base = tid + dil * half;
  T xc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) xc[v] = X[base + NT * v];
#pragma unroll
  for (int s = 0; s < SG; ++s) {
    const T h0 = s < ns ? taps[((s0 + s) * (half + 1)) * C] : T(0);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      re[v][s] = h0 * xc[v];
      im[v][s] = T(0);
    }
  }
  // per-scale rows of the tap table (scalar registers, fixed over the tap loop) and one 32-bit
  // byte offset shared by all of them: a scalar load per scale and tap with the offset in a
  // register, instead of a 64-bit address rebuilt per scale and tap
  const char* trow[SG];
#pragma unroll
  for (int s = 0; s < SG; ++s)
    trow[s] = reinterpret_cast<const char*>(taps + (int64_t)(s0 + min(s, ns - 1)) * (half + 1) * C);
  for (int t = 1; t <= tmax; ++t) {
    const unsigned toff = (unsigned)(t * C * (int)sizeof(T));
    T ps[V], ms[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const T a = X[base + NT * v - dil * t];
      const T b = X[base + NT * v + dil * t];
      ps[v] = a + b;
      ms[v] = a - b;
    }
#pragma unroll
    for (int s = 0; s < SG; ++s) {
      if (s < ns) {
        const T* tp = reinterpret_cast<const T*>(trow[s] + toff);
        const T hr = tp[0];
#pragma unroll
        for (int v = 0; v < V; ++v) re[v][s] = fma(hr, ps[v], re[v][s]);
        if (CPLX) {
          const T hi = tp[1];
#pragma unroll
          for (int v = 0; v < V; ++v) im[v][s] = fma(hi, ms[v], im[v][s]);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ bank forward
template <typename T, bool CPLX>
__global__ void __launch_bounds__(NT) morlet_forward_kernel(Stage st, T* __restrict__ y,
                                                            int s_total, int tiles) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* X = reinterpret_cast<T*>(smem_raw);
  constexpr int C = CPLX ? 2 : 1;
  const int64_t row = blockIdx.x / tiles;
  const int64_t n0 = (int64_t)(blockIdx.x % tiles) * TT;
  const int span = TT + 2 * st.dil * st.half;
  const T* xrow = static_cast<const T*>(st.x) + row * st.n_in;
  stage_row(X, xrow, n0 + st.x_off - (int64_t)st.dil * st.half, span, st.n_in);
  __syncthreads();
  const T* taps = static_cast<const T*>(st.taps);
  for (int s0 = 0; s0 < st.n_scales; s0 += SG) {
    const int ns = min(SG, st.n_scales - s0);
    T re[V][SG], im[V][SG];
    bank_group<T, CPLX>(X, taps, st.half, st.dil, s0, ns, st.sup[s0 + ns - 1], re, im);
#pragma unroll
    for (int s = 0; s < SG; ++s) {
      if (s >= ns) break;
      T* yrow = y + ((row * s_total + st.chan[s0 + s]) * st.n_out) * C;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int64_t n = n0 + threadIdx.x + NT * v;
        if (n < st.n_out) {
          if (CPLX) {
            typedef T v2 __attribute__((ext_vector_type(2)));
            *reinterpret_cast<v2*>(yrow + 2 * n) = v2{re[v][s], im[v][s]};
          } else {
            yrow[n] = re[v][s];
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ bank adjoint (grad x)
// gx[p] (+)= sum_s [h_s[0] g_re[q] + sum_t h_s[t] (g_re[q + dil t] + g_re[q - dil t])
//                                  + g_s[t] (g_im[q + dil t] - g_im[q - dil t])],  q = p - x_off
// g: (rows, g_scales, n_out, C) with local scale s at channel chan[s].
template <typename T, bool CPLX>
__global__ void __launch_bounds__(NT) morlet_backward_x_kernel(Stage st, const T* __restrict__ g,
                                                               T* __restrict__ gx, int g_scales,
                                                               int tiles, int accumulate) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* G = reinterpret_cast<T*>(smem_raw);  // one scale: span x C (interleaved)
  constexpr int C = CPLX ? 2 : 1;
  const int64_t row = blockIdx.x / tiles;
  const int64_t p0 = (int64_t)(blockIdx.x % tiles) * TT;
  const int half = st.half, dil = st.dil;
  const int span = TT + 2 * dil * half;
  const int64_t q0 = p0 - st.x_off - (int64_t)dil * half;  // g position of G[0]
  const T* taps = static_cast<const T*>(st.taps);
  const int tid = threadIdx.x;
  const int nel = span * C;
  T acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = T(0);
  // The g tile of the next scale is loaded into registers while the current one is used (its
  // first GPF * NT elements; a longer tile loads the rest when it is staged).
  constexpr int GPF = sizeof(T) == 8 ? 4 : 8;
  T gr[GPF];
  auto fetch = [&](int s) {
    const T* grow = g + ((row * g_scales + st.chan[s]) * st.n_out) * C;
#pragma unroll
    for (int r = 0; r < GPF; ++r) {
      const int k = tid + r * NT;
      if (r * NT < nel) {
        const int64_t q = q0 + k / C;
        gr[r] = grow[min(max(q, (int64_t)0), st.n_out - 1) * C + (k % C)];
      }
    }
  };
  if (st.n_scales > 0) fetch(0);
  for (int s = 0; s < st.n_scales; ++s) {
    const T* grow = g + ((row * g_scales + st.chan[s]) * st.n_out) * C;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < GPF; ++r) {
      const int k = tid + r * NT;
      if (r * NT < nel && k < nel) {
        const int64_t q = q0 + k / C;
        G[k] = (q >= 0 && q < st.n_out) ? gr[r] : T(0);
      }
    }
    for (int k = GPF * NT + tid; k < nel; k += NT) {
      const int64_t q = q0 + k / C;
      const T w = grow[min(max(q, (int64_t)0), st.n_out - 1) * C + (k % C)];
      G[k] = (q >= 0 && q < st.n_out) ? w : T(0);
    }
    __syncthreads();
    if (s + 1 < st.n_scales) fetch(s + 1);
    const int tmax = st.sup[s];
    const T* tp = taps + s * (half + 1) * C;
    const int base = tid + dil * half;
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = fma(tp[0], G[(base + NT * v) * C], acc[v]);
    for (int t = 1; t <= tmax; ++t) {
      const T hr = tp[t * C];
      const T hi = CPLX ? tp[t * C + 1] : T(0);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int iu = (base + NT * v + dil * t) * C;
        const int id = (base + NT * v - dil * t) * C;
        acc[v] = fma(hr, G[iu] + G[id], acc[v]);
        if (CPLX) acc[v] = fma(hi, G[iu + 1] - G[id + 1], acc[v]);
      }
    }
  }
  T* gxrow = gx + row * st.n_in;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t p = p0 + tid + NT * v;
    if (p < st.n_in) gxrow[p] = accumulate ? gxrow[p] + acc[v] : acc[v];
  }
}

// ------------------------------------------------------------------ bank adjoint, windowed
// The same adjoint for a power-of-two dilation, computed only where g reaches: gx[p] has a
// contribution iff p - x_off lies in [-dil half, n_out - 1 + dil half], so the tiles cover
// [lo, hi) = that range clipped to [0, n_in); positions outside it are left alone
// (accumulate) or zeroed.
//
// Positions are p = lo + R + dil j (residue R < dil, j >= 0).  A tile takes D of the dil
// residue classes (R0 .. R0 + D - 1) and J = TT / D consecutive j of each, and stages their
// g values interleaved: tile element i = R_local + D jj holds g at q = lo - x_off + R0 +
// R_local + dil (j0 + jj - H), jj < J + 2 H (H = half rounded up to RUN).  Neighbours in a
// residue class are D apart in the tile, so the tap loop is the same for every dilation and
// a small D keeps the halo (2 H D elements per tile) small next to the TT outputs.
//
// Thread (r, b) = (tid % D, tid / D) owns the RUN outputs j = j0 + RUN b + k, k < RUN, of
// residue R0 + r.  With U_m = G[q_0 + D m] (q_0 = D H + r + D RUN b) output k needs U_{k+t}
// and U_{k-t} at tap t, so two RUN-slot register windows (up: U_t .. U_{t+RUN-1}, down:
// U_{-t} .. U_{RUN-1-t}) serve every output of the thread, and each tap loads just two new
// values (one per window) into the slot the tap frees; the tap loop is unrolled by RUN so
// every slot index is a compile-time constant.
//
// LDS layout: tile element i lives at phys(i) = i + D floor(i / (D RUN)), one step of
// padding per thread run.  Because H is a multiple of RUN the runs align to that grid, so
// phys(q_0 + D m) = phys(q_0) + D (m + floor(m / RUN)): loads are a per-thread base plus
// immediate offsets, and the 32 lanes of a half-wave read 8-byte words in distinct banks for
// every D (lane stride RUN + 1 words for D = 1).
constexpr int RUN = V;  // outputs per thread; TT = NT RUN

template <int D>
__device__ inline int adj_phys(int i) {
  constexpr int SH = __builtin_ctz(D * RUN);
  return i + D * (i >> SH);
}

template <typename T, bool CPLX, int D>
__global__ void __launch_bounds__(NT) morlet_adjoint_kernel(Stage st, const T* __restrict__ g,
                                                            T* __restrict__ gx, int g_scales,
                                                            int tiles, int jblocks, int64_t lo,
                                                            int64_t hi, int H, int accumulate) {
  static_assert(NT % D == 0, "a residue class needs whole thread runs");
  constexpr int J = TT / D;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* G = reinterpret_cast<T*>(smem_raw);
  constexpr int C = CPLX ? 2 : 1;
  const int64_t dil = st.dil;
  const int64_t row = blockIdx.x / tiles;
  const int tile = (int)(blockIdx.x % tiles);
  const int64_t R0 = (int64_t)(tile / jblocks) * D;
  const int64_t j0 = (int64_t)(tile % jblocks) * J;
  const int nel = D * (J + 2 * H) * C;
  const int64_t qbase = lo - st.x_off + R0 + dil * (j0 - H);  // g position of element 0
  const T* taps = static_cast<const T*>(st.taps);
  const int tid = threadIdx.x;
  T* gxrow = gx + row * st.n_in;
  if (!accumulate) {  // zero the positions g does not reach, spread over the row's tiles
    const int64_t outside = lo + (st.n_in - hi);
    for (int64_t j = (int64_t)tile * NT + tid; j < outside; j += (int64_t)tiles * NT)
      gxrow[j < lo ? j : hi + (j - lo)] = T(0);
  }
  T acc[RUN];
#pragma unroll
  for (int k = 0; k < RUN; ++k) acc[k] = T(0);
  // g is read through a buffer resource per (row, scale) plane: byte offsets are 32-bit (the
  // host takes this kernel only when every g position a tile touches, -2 dil H .. n_out +
  // 2 dil H, is within 2^31 bytes of the plane) and positions outside [0, n_out) read as 0.
  const int qb = (int)qbase;
  const int dl = (int)dil;
  auto goff = [&](int k) -> int {
    const int i = k / C;
    return ((qb + (i % D) + dl * (i / D)) * C + (k % C)) * (int)sizeof(T);
  };
  auto plane = [&](int s) {
    return make_rsrc(g + ((row * g_scales + st.chan[s]) * st.n_out) * C,
                     st.n_out * C * (int64_t)sizeof(T));
  };
  constexpr int GPF = sizeof(T) == 8 ? 4 : 8;
  T gr[GPF];
  auto fetch = [&](int s) {
    const BufRsrc pr = plane(s);
#pragma unroll
    for (int e = 0; e < GPF; ++e)
      if (e * NT < nel) gr[e] = buf_load<T>(pr, goff(tid + e * NT));
  };
  const int r = tid % D, b = tid / D;
  const int pb = adj_phys<D>(D * H + r + D * RUN * b);  // phys of U_0
  if (st.n_scales > 0) fetch(0);
  for (int s = 0; s < st.n_scales; ++s) {
    __syncthreads();
#pragma unroll
    for (int e = 0; e < GPF; ++e) {
      const int k = tid + e * NT;
      if (e * NT < nel && k < nel) G[adj_phys<D>(k / C) * C + (k % C)] = gr[e];
    }
    {  // the rest of the tile: SB loads per thread in flight before their LDS writes
      constexpr int SB = 4;
      const BufRsrc pr = plane(s);
      for (int k0 = GPF * NT + tid; k0 < nel; k0 += SB * NT) {
        T v[SB];
#pragma unroll
        for (int e = 0; e < SB; ++e) v[e] = buf_load<T>(pr, goff(k0 + e * NT));
#pragma unroll
        for (int e = 0; e < SB; ++e) {
          const int k = k0 + e * NT;
          if (k < nel) G[adj_phys<D>(k / C) * C + (k % C)] = v[e];
        }
      }
    }
    __syncthreads();
    if (s + 1 < st.n_scales) fetch(s + 1);
    const int tmax = st.sup[s];
    const T* tp = taps + s * (st.half + 1) * C;
    T upr[RUN], upi[RUN], dnr[RUN], dni[RUN];
    {
      const T h0 = tp[0];
#pragma unroll
      for (int k = 0; k < RUN; ++k) {
        const T* e = G + (pb + D * k) * C;
        upr[k] = dnr[k] = e[0];
        if (CPLX) upi[k] = dni[k] = e[1];
        acc[k] = fma(h0, upr[k], acc[k]);
      }
    }
    for (int t0 = 1, blk = 0; t0 <= tmax; t0 += RUN, ++blk) {
      const T* ub = G + (pb + D * (RUN + 1) * blk) * C;
      const T* db = G + (pb - D * (RUN + 1) * blk) * C;
#pragma unroll
      for (int u = 0; u < RUN; ++u) {
        if (t0 + u <= tmax) {
          // U_{t-1+RUN} into up slot u, U_{-t} into down slot RUN-1-u (t = t0 + u)
          const T* eu = ub + D * (u + RUN + 1) * C;
          const T* ed = db - D * (u + 2) * C;
          upr[u] = eu[0];
          dnr[RUN - 1 - u] = ed[0];
          if (CPLX) {
            upi[u] = eu[1];
            dni[RUN - 1 - u] = ed[1];
          }
          const T hr = tp[(t0 + u) * C];
          const T hi_ = CPLX ? tp[(t0 + u) * C + 1] : T(0);
#pragma unroll
          for (int k = 0; k < RUN; ++k) {
            const int a = (k + 1 + u) % RUN, c = (k + 2 * RUN - 1 - u) % RUN;
            acc[k] = fma(hr, upr[a] + dnr[c], acc[k]);
            if (CPLX) acc[k] = fma(hi_, upi[a] - dni[c], acc[k]);
          }
        }
      }
    }
  }
  if (R0 + r < dil) {
#pragma unroll
    for (int k = 0; k < RUN; ++k) {
      const int64_t p = lo + R0 + r + dil * (j0 + RUN * b + k);
      if (p < hi) gxrow[p] = accumulate ? gxrow[p] + acc[k] : acc[k];
    }
  }
}

// ------------------------------------------------------------------ filter gradient
// Partial sums per workgroup of  gh[s][k][ch] = sum_n g[s, n, ch] x[n + x_off - dil (k - half)]
// for k = 0 .. 2 half (every tap, no symmetry assumed).  partial: (n_el, blocks) with
// n_el = n_scales (2 half + 1) C, written transposed so that the final reduction reads
// contiguous memory.
//
// Register tiling: g of up to HS scales is staged in LDS next to the x tile; each wave takes
// blocks of HB taps, and each lane HP consecutive positions at a time, so one 16-byte LDS read
// of x feeds HP positions x C channels x HS scales FMAs (for dil <= 2 the taps of a block
// share one window of x, read once).  Lane l handles positions HP l + 64 HP q; at the end the
// HS HB C sums of a lane are reduced over the 64 lanes of the wave by a butterfly that halves
// the values per lane at every step (reduce-scatter), then written by the lanes that hold them.
constexpr int HB = 8;   // taps per block
constexpr int HS4 = 4;  // scales per group (largest)
constexpr int HP = 4;   // consecutive positions per lane and step
constexpr int HPAD = 16;  // zeros in front of the x tile (window reads of clamped taps)

// One step of butterfly_sum: with offset O and W values per lane, a lane keeps the half of
// its values selected by (lane & O), summed with its partner's copy of that half.
template <typename T, int O, int W>
__device__ inline void butterfly_step(T (&v)[64], int lane) {
  if constexpr (O > 0) {
    if constexpr (W > 1) {
      const bool hi = lane & O;
#pragma unroll
      for (int j = 0; j < W / 2; ++j) {
        const T send = hi ? v[j] : v[j + W / 2];
        const T keep = hi ? v[j + W / 2] : v[j];
        v[j] = keep + __shfl_xor(send, O);
      }
      butterfly_step<T, O / 2, W / 2>(v, lane);
    } else {
      v[0] += __shfl_xor(v[0], O);
      butterfly_step<T, O / 2, 1>(v, lane);
    }
  }
}

// Sum W values per lane over the 64 lanes of a wave, leaving one sum per lane (v[0]).
template <typename T, int W>
__device__ inline void butterfly_sum(T (&v)[64], int lane) {
  butterfly_step<T, 32, W>(v, lane);
}

// Index of the value a lane holds after butterfly_sum over W values: the bits of the lane
// picked by the halving steps (offsets 32, 16, ..) read from the most significant side.
template <int W>
__device__ inline int butterfly_index(int lane) {
  int idx = 0;
#pragma unroll
  for (int o = 32, w = W; o > 0 && w > 1; o >>= 1, w >>= 1) idx = 2 * idx + ((lane & o) ? 1 : 0);
  return idx;
}

// One launch handles the scales [s_begin, s_end) in groups of HS (4, 2 or 1): the host
// launches the last n_scales % 4 scales with a smaller HS, so no group computes empty scales.
// partial holds rows from scale s_part on: tap k of scale s, channel ch, is row
// ((s - s_part) K + k) C + ch, one column per workgroup.
template <typename T, bool CPLX, int DIL, int HS>  // DIL: 1, 2, or 0 for any multiple of 4
__global__ void __launch_bounds__(NT) morlet_backward_h_kernel(Stage st, const T* __restrict__ g,
                                                               T* __restrict__ partial,
                                                               int g_scales, int tiles,
                                                               int s_begin, int s_end,
                                                               int s_part) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int C = CPLX ? 2 : 1;
  constexpr int NV = HS * HB * C;  // sums per lane (a power of two)
  static_assert((NV & (NV - 1)) == 0 && NV <= 64, "butterfly needs a power of two <= 64");
  T* const X = reinterpret_cast<T*>(smem_raw) + HPAD;  // X[-HPAD..-1] = 0
  const int half = st.half, dil = DIL > 0 ? DIL : st.dil;
  const int span = TT + 2 * dil * half;
  T* const G = X + ((span + 4 + 3) & ~3);  // G[(sl C + ch) TT + i], HS scales
  const int64_t row = blockIdx.x / tiles;
  const int64_t n0 = (int64_t)(blockIdx.x % tiles) * TT;
  const int64_t nblocks = (int64_t)gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const T* xrow = static_cast<const T*>(st.x) + row * st.n_in;
  if (tid < HPAD) X[tid - HPAD] = T(0);
  stage_row(X, xrow, n0 + st.x_off - (int64_t)dil * half, span + 4, st.n_in);
  const int K = 2 * half + 1;
  const int nvalid = (int)min((int64_t)TT, st.n_out - n0);
  typedef T v4 __attribute__((ext_vector_type(4)));
  const int nq = (nvalid + 64 * HP - 1) / (64 * HP);  // position steps holding valid g
  for (int s0 = s_begin; s0 < s_end; s0 += HS) {
    const int ns = min(HS, s_end - s0);
    __syncthreads();
    for (int k = tid; k < HS * TT * C; k += NT) {
      const int sl = k / (TT * C), r = k % (TT * C), i = r / C, ch = r % C;
      T v = T(0);
      if (sl < ns && i < nvalid)
        v = g[((row * g_scales + st.chan[s0 + sl]) * st.n_out + n0) * C + r];
      G[(sl * C + ch) * TT + i] = v;
    }
    __syncthreads();
    for (int k0 = wave * HB; k0 < K; k0 += (NT / 64) * HB) {
      T acc[HS][HB][C];
#pragma unroll
      for (int a = 0; a < HS; ++a)
#pragma unroll
        for (int b = 0; b < HB; ++b)
#pragma unroll
          for (int ch = 0; ch < C; ++ch) acc[a][b][ch] = T(0);
      for (int q = 0; q < nq; ++q) {
        const int i = (q * 64 + lane) * HP;
        T gv[HS][C][HP];
#pragma unroll
        for (int a = 0; a < HS; ++a)
#pragma unroll
          for (int ch = 0; ch < C; ++ch) {
            const v4 w = *reinterpret_cast<const v4*>(G + (a * C + ch) * TT + i);
#pragma unroll
            for (int p = 0; p < HP; ++p) gv[a][ch][p] = w[p];
          }
        if constexpr (DIL > 0) {
          // taps k0 .. k0 + HB - 1 read x[i + p + DIL (2 half - k)]: one window of
          // HP + DIL (HB - 1) values starting at i + DIL (2 half - k0 - HB + 1)
          constexpr int NW = HP + DIL * (HB - 1);
          const T* xw = X + i + DIL * (2 * half - k0 - (HB - 1));
          T wv[NW];
#pragma unroll
          for (int m = 0; m < NW; ++m) wv[m] = xw[m];
#pragma unroll
          for (int b = 0; b < HB; ++b)
#pragma unroll
            for (int p = 0; p < HP; ++p) {
              const T xv = wv[p + DIL * (HB - 1 - b)];
#pragma unroll
              for (int a = 0; a < HS; ++a)
#pragma unroll
                for (int ch = 0; ch < C; ++ch) acc[a][b][ch] = fma(gv[a][ch][p], xv, acc[a][b][ch]);
            }
        } else {
#pragma unroll
          for (int b = 0; b < HB; ++b) {
            const int k = min(k0 + b, K - 1);
            const v4 w = *reinterpret_cast<const v4*>(X + i + dil * (2 * half - k));
#pragma unroll
            for (int p = 0; p < HP; ++p)
#pragma unroll
              for (int a = 0; a < HS; ++a)
#pragma unroll
                for (int ch = 0; ch < C; ++ch) acc[a][b][ch] = fma(gv[a][ch][p], w[p], acc[a][b][ch]);
          }
        }
      }
      // positions beyond nvalid have g = 0 and add nothing
      T v[64];
#pragma unroll
      for (int a = 0; a < HS; ++a)
#pragma unroll
        for (int b = 0; b < HB; ++b)
#pragma unroll
          for (int ch = 0; ch < C; ++ch) v[(a * HB + b) * C + ch] = acc[a][b][ch];
      butterfly_sum<T, NV>(v, lane);
      // the lanes holding value j: lane bits picked by the halving steps; with NV < 64 the
      // remaining steps left several lanes with the same sum, and the first of them writes
      const int j = butterfly_index<NV>(lane);
      const int rest = 64 / NV;  // lanes sharing one sum: those differing in the low bits
      if ((lane & (rest - 1)) == 0) {
        const int a = j / (HB * C), b = (j / C) % HB, ch = j % C;
        const int k = k0 + b;
        if (a < ns && k < K)
          partial[((int64_t)((s0 + a - s_part) * K + k) * C + ch) * nblocks + blockIdx.x] = v[0];
      }
    }
  }
}

// float -> bf16 bits, round to nearest even (NaN stays a NaN)
__device__ inline uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// ------------------------------------------------------------------ filter gradient, MFMA
// The same partial sums as a matrix product on the matrix cores:
//     gh[(s, ch)][k] = sum_n G[(s, ch)][n] X[n][k],   X[n][k] = x[n + x_off - dil (k - half)]
// with one v_mfma_*_16x16x4 per 4 positions and 16 taps: A = G (16 rows = up to 16 / C
// scales x C channels, 4 positions), B = X (4 positions x 16 taps), accumulated in the
// instruction's 16 x 16 result for every tap block of the stage (K <= 16 MB_KB).
// Operand layout (16x16x4, one block): lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16];
// result element e of lane l is D[row][l % 16] with row = 4 (l / 16) + e for f32 and
// (l / 16) + 4 e for f64 (both measured on gfx950).
//
// A workgroup loops over position tiles (row, n0) with stride gridDim.x, so the sums stay in
// the result registers over several tiles; each wave takes a quarter of every tile.  G comes
// straight from global memory (each element is read once); the x tile (TT + 2 dil half + 4
// samples) is staged in LDS with four words of skew per dil words (dil >= 8), so the 16 taps
// of an instruction (addresses dil apart) fall in distinct banks.  At the end the four waves' sums are added in
// LDS and the workgroup writes column blockIdx.x of `partial` (n_el x gridDim.x).
// With BF (fp32 storage, the reference's "bf16" precision, conv.py:372-408) both operands are
// rounded to bf16 (round to nearest even, v_cvt_pk_bf16_f32) and each
// v_mfma_f32_16x16x16_bf16 takes 16 positions: lane l supplies
// A[l % 16][4 (l / 16) + v] and B[4 (l / 16) + v][l % 16], v < 4 (four consecutive positions,
// which never straddle a skew step: the skew period dil is a multiple of 8), with the same
// result layout; sums stay fp32.
constexpr int MB_KB = 8;   // tap blocks of 16 (K <= 128)
constexpr int MB_U = 8;    // instructions per A prefetch chunk (TT / 4 is a multiple of 4 MB_U)
constexpr int MB_XR = 1;   // x window registers per thread (the first MB_XR NT samples)
#ifndef GH_VEC_SCALES
#define GH_VEC_SCALES 1  // trailing scale groups this small skip the matrix cores
#endif

template <typename T>
struct Mfma16;
template <>
struct Mfma16<float> {
  typedef float v4 __attribute__((ext_vector_type(4)));
  static __device__ inline v4 mma(float a, float b, v4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ inline int row(int lane, int e) { return 4 * (lane / 16) + e; }
};
template <>
struct Mfma16<double> {
  typedef double v4 __attribute__((ext_vector_type(4)));
  static __device__ inline v4 mma(double a, double b, v4 c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  static __device__ inline int row(int lane, int e) { return lane / 16 + 4 * e; }
};

template <typename T, bool CPLX, int KB, bool BF, bool LIN>  // KB = ceil(K / 16) tap blocks
__global__ void __launch_bounds__(NT) morlet_grad_h_mfma_kernel(Stage st, const T* __restrict__ g,
                                                                T* __restrict__ partial,
                                                                int g_scales, int tiles,
                                                                int64_t total, int s_begin,
                                                                int s_end, int sk) {
  constexpr int kblocks = KB;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  typedef typename Mfma16<T>::v4 v4;
  constexpr int C = CPLX ? 2 : 1;
  T* const X = reinterpret_cast<T*>(smem_raw);
  // (the wave index made visibly wave-uniform: chunk bounds, the tile choice and with it the
  // A buffer resource stay in scalar registers)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = st.half, dil = st.dil, K = 2 * half + 1;
  const int span = TT + 2 * dil * half + 4;
  const int ns = s_end - s_begin;
  const int arow = lane & 15, asl = arow / C, ach = arow % C;
  const bool arow_ok = asl < ns;
  const int chan_a = arow_ok ? st.chan[s_begin + asl] : 0;
  const int kpos = lane >> 4;  // position of this lane within an instruction's four
  // skewed LDS index of x element i: i + 4 (i >> sk) with 2^sk = dil (no skew below dil 8).
  // Tap offsets are multiples of dil, so skew(p + off) = skew(p) + skew(off); consecutive taps
  // are dil + 4 words apart, i.e. 4 banks (mod 64) for every power-of-two dil, so the 16 taps
  // x 4 positions of an instruction's B operand fall in 64 distinct banks.
  auto skew = [sk](int i) { return i + ((i >> sk) << 2); };
  int boff[KB];                // skewed x offset of this lane's tap in every block
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) boff[kb] = skew(dil * (2 * half - min(kb * 16 + arow, K - 1)));
  v4 acc[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) acc[kb] = v4{T(0), T(0), T(0), T(0)};
  // Software pipeline over the workgroup's tiles: the x window of the next tile is loaded into
  // registers (its first MB_XR NT samples) while the current tile is multiplied, and the last
  // A chunk of a tile is followed by the first chunk of the next tile.  Loads are unconditional
  // from clamped (valid) indices; masks are applied where the values are used.
  // each tile's valid positions, in chunks of 4 MB_U, split evenly over the four waves (a full
  // tile: a quarter each; a row's last, partial tile: no idle wave)
  auto wave_range = [&](int nvalid, int& b, int& e) {
    const int chunk = 4 * MB_U;
    const int per = ((nvalid + chunk - 1) / chunk + 3) / 4 * chunk;
    b = min(wave * per, nvalid);
    e = min(b + per, nvalid);
  };
  // A comes through a buffer resource per tile whose base is the tile's first position in the
  // row's block of g (wave-uniform); a lane's 32-bit offset selects its scale row and channel,
  // and the slots of a chunk differ by constants (immediate offsets).  The host keeps every
  // offset below 2^31; the resource ends with g, so reads past a row's last valid position
  // return finite data of g or 0, and are masked below.  Rows of scales >= ns load row 0 and
  // are never masked: their result rows are discarded.
  struct Tile {
    BufRsrc ga;     // g from the tile's first position of the row block
    const T* xrow;
    int64_t xb;     // x index of window element 0
    int nvalid;
  };
  const int64_t g_elems = (total / tiles) * g_scales * st.n_out * C;
  auto tile_of = [&](int64_t t) {
    Tile q;
    const int64_t row = t / tiles, n0 = (t % tiles) * (int64_t)TT;
    const int64_t e0 = row * g_scales * st.n_out * C + n0 * C;
    q.ga = make_rsrc(g + e0, min((g_elems - e0) * (int64_t)sizeof(T), (int64_t)INT32_MAX));
    q.xrow = static_cast<const T*>(st.x) + row * st.n_in;
    q.xb = n0 + st.x_off - (int64_t)dil * half;
    q.nvalid = (int)min((int64_t)TT, st.n_out - n0);
    return q;
  };
  T an[MB_U], xr[MB_XR];
  // position of prefetch slot u of a chunk starting at c0 (this lane's A elements), and the
  // lane's part of it
  auto a_pos = [&](int c0, int u) {
    return BF ? c0 + 16 * (u / 4) + 4 * kpos + (u % 4) : c0 + 4 * u + kpos;
  };
  const int a_lane =
      (int)(((int64_t)chan_a * st.n_out + (BF ? 4 : 1) * kpos) * C + ach) * (int)sizeof(T);
  auto load_a = [&](const Tile& q, int c0) {
    const int voff = a_lane + c0 * C * (int)sizeof(T);
#pragma unroll
    for (int u = 0; u < MB_U; ++u)
      an[u] = buf_load<T>(q.ga, voff + (a_pos(0, u) - a_pos(0, 0)) * C * (int)sizeof(T));
  };
  // B addresses (LIN, chosen by the host when sk >= 5): within a chunk (32 positions from a
  // multiple of 32) the skewed index is linear when the skew period dil is >= 32 or there is
  // no skew, so the slots' LDS reads differ by constants (immediate offsets) from one address
  // per tap block
  auto load_x = [&](const Tile& q) {
#pragma unroll
    for (int r = 0; r < MB_XR; ++r)
      xr[r] = q.xrow[min(max(q.xb + tid + r * NT, (int64_t)0), st.n_in - 1)];
  };
  int64_t t = blockIdx.x;
  Tile cur_t = tile_of(t < total ? t : 0);
  load_x(cur_t);
  int pbeg, pend;
  wave_range(cur_t.nvalid, pbeg, pend);
  load_a(cur_t, pbeg);
  for (; t < total; t += gridDim.x) {
    const Tile nxt = tile_of(t + gridDim.x < total ? t + gridDim.x : t);
    __syncthreads();  // the previous tile's reads of X are done
#pragma unroll
    for (int r = 0; r < MB_XR; ++r) {
      const int i = tid + r * NT;
      const int64_t xi = cur_t.xb + i;
      if (i < span) X[skew(i)] = (xi >= 0 && xi < st.n_in) ? xr[r] : T(0);
    }
    batched_copy<T>(
        MB_XR * NT, span,
        [&](int i) { return cur_t.xrow[min(max(cur_t.xb + i, (int64_t)0), st.n_in - 1)]; },
        [&](int i, T w) {
          const int64_t xi = cur_t.xb + i;
          X[skew(i)] = (xi >= 0 && xi < st.n_in) ? w : T(0);
        });
    __syncthreads();
    load_x(nxt);
    const int nvalid = cur_t.nvalid;
    int nbeg, nend;
    wave_range(nxt.nvalid, nbeg, nend);
    if (pbeg >= pend) load_a(nxt, nbeg);  // no positions of this tile for this wave
    for (int c0 = pbeg; c0 < pend; c0 += 4 * MB_U) {
      // positions >= nvalid (a row's last tile only) get a zero A element
      const bool full = c0 + 4 * MB_U <= nvalid;
      if constexpr (BF) {
        typedef short v4s __attribute__((ext_vector_type(4)));
        v4s a4[MB_U / 4];
#pragma unroll
        for (int u = 0; u < MB_U; ++u)
          a4[u / 4][u % 4] = __builtin_bit_cast(
              short, (__bf16)((full || a_pos(c0, u) < nvalid) ? (float)an[u] : 0.f));
        const bool last = c0 + 4 * MB_U >= pend;
        load_a(last ? nxt : cur_t, last ? nbeg : c0 + 4 * MB_U);
        const int xl = skew(c0 + 4 * kpos);
#pragma unroll
        for (int u2 = 0; u2 < MB_U / 4; ++u2) {
          const T* xp = LIN ? X + (xl + 16 * u2) : X + skew(c0 + 16 * u2 + 4 * kpos);
          v4s b[KB];
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              b[kb][v] = __builtin_bit_cast(short, (__bf16)(float)xp[boff[kb] + v]);
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
            acc[kb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a4[u2], b[kb], acc[kb], 0, 0, 0);
        }
        continue;
      }
      T cur[MB_U];
      if (full) {
#pragma unroll
        for (int u = 0; u < MB_U; ++u) cur[u] = an[u];
      } else {
#pragma unroll
        for (int u = 0; u < MB_U; ++u) cur[u] = c0 + 4 * u + kpos < nvalid ? an[u] : T(0);
      }
      const bool last = c0 + 4 * MB_U >= pend;
      load_a(last ? nxt : cur_t, last ? nbeg : c0 + 4 * MB_U);
      // B values: the LDS reads of step u + 1 are issued before the instructions of step u,
      // so an instruction never waits for its own read (fences keep that order; without them
      // the compiler reuses one register and puts a full LDS wait before every instruction)
      const T* xl[KB];  // LIN: slot u of tap block kb reads xl[kb][4 u]
      const int x0 = skew(c0 + kpos);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) xl[kb] = X + (x0 + boff[kb]);
      T bc[KB], bn[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) bc[kb] = xl[kb][0];
#pragma unroll
      for (int u = 0; u < MB_U; ++u) {
        if (u + 1 < MB_U) {
          if constexpr (LIN) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) bn[kb] = xl[kb][4 * (u + 1)];
          } else {
            const T* xp = X + skew(c0 + 4 * (u + 1) + kpos);
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) bn[kb] = xp[boff[kb]];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) acc[kb] = Mfma16<T>::mma(cur[u], bc[kb], acc[kb]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) bc[kb] = bn[kb];
      }
    }
    cur_t = nxt;
    pbeg = nbeg;
    pend = nend;
  }
  // add the four waves' sums (X is free now) and write this workgroup's column
  __syncthreads();
  T* const red = X;  // [wave][kb][e][lane]
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
    for (int e = 0; e < 4; ++e) red[((wave * kblocks + kb) * 4 + e) * 64 + lane] = acc[kb][e];
  }
  __syncthreads();
  const int64_t ncols = gridDim.x;
  for (int idx = tid; idx < kblocks * 256; idx += NT) {
    T v = T(0);
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) v += red[w * kblocks * 256 + idx];
    const int kb = idx / 256, e = (idx / 64) % 4, l = idx % 64;
    const int i = Mfma16<T>::row(l, e), sl = i / C, ch = i % C, k = kb * 16 + (l % 16);
    if (sl < ns && k < K)
      partial[((int64_t)((s_begin + sl) * K + k) * C + ch) * ncols + blockIdx.x] = v;
  }
}

// ------------------------------------------------------------------ bank adjoint, matrix cores
// The adjoint as a matrix product.  Positions p = lo + rho + dil i (residue rho < dil) of a
// row see g only at q = lo - x_off + rho + dil j, so with
//     u_{rho,s,c}[j] = g[r, chan_s, lo - x_off + rho + dil j, c]   (0 outside [0, n_out))
// and the full filters F_{s,c}[k], |k| <= sup_s (F_{s,0}[k] = taps[s][|k|][0] and F_{s,1}[k] =
// sign(k) taps[s][|k|][1]: the even and odd Morlet halves of the compact taps)
//     gx[r, lo + rho + dil i] = sum_{s,c} sum_k F_{s,c}[k] u_{rho,s,c}[i + k].
// The filter does not depend on the row or the residue, so for 16 lines m = (row, residue) and
// 16 consecutive i this is U (16 lines x 16 + 2 sup_s window positions) times the banded
// Toeplitz matrix Z[j][i] = F[j - i - sup_s] (window x 16 outputs), accumulated over (s, c) in
// the result registers of one v_mfma_*_16x16x4 per 4 window positions j = 4 t + kap (A: lane l
// gives U[l % 16][4 t + l / 16]; B: Z[4 t + l / 16][l % 16]).  Z is the same for every tile,
// so a wave reads it once per step for its MA_NB tiles.
//
// The 16 lines of a workgroup are 16 / D rows x D consecutive residues rho0 .. rho0 + D - 1
// (D = min(dil, 16)), so a row's staged positions rho0 + rho + dil j are runs of D consecutive
// g positions: whole cache lines from D = 16 on, one contiguous range for dil <= 16.  A
// workgroup takes MA_TI = 4 MA_NB 16 consecutive i (MA_NB tiles per wave); consecutive
// workgroups take consecutive residue blocks.  Per scale it stages u of both channels over the
// tiles' window (MA_TI + 2 sup_s + 3 <= MA_WL positions; the last 3 meet only zero taps) in
// LDS, lines WS words apart with WS = 4 (mod 32), so the 64 lanes of an A read (16 lines x 4
// consecutive j) and of a staging store (D lines x 64 / D consecutive j) hit distinct banks;
// and the scale's zero-padded filters.  The whole window of the next scale is loaded into
// registers (MA_PFN loads per thread, through a buffer resource per (row, scale) plane:
// positions outside [0, n_out), and rows past the last, read 0) while the current scale is
// multiplied.
constexpr int MA_NB = 2;               // 16 x 16 tiles per wave
constexpr int MA_TI = 4 * 16 * MA_NB;  // outputs per line of a workgroup
constexpr int MA_WL = 256;             // longest staged window (half <= (MA_WL - MA_TI - 3) / 2)
constexpr int MA_PFN = 16 * MA_WL / NT;  // prefetch loads per thread (16 lines x MA_WL)

// bf16 operands (fp32 storage and accumulation): one v_mfma_f32_16x16x16_bf16 per 16 window
// positions, so the window is staged 12 positions longer (MA_TI + 2 sup + 15), in bf16.
// LDS line stride (elements) of the staged u, length of an fp32 filter table, and (bf16) the
// steps of the B-operand table, for a stage's half
__host__ __device__ inline int ma_ext(bool bf) { return bf ? 15 : 3; }
__host__ __device__ inline int ma_ws(int half, bool bf = false) {
  return 32 * ((MA_TI + 2 * half + ma_ext(bf) - 4 + 31) / 32) + 4;
}
__host__ __device__ inline int ma_fl(int half, bool bf = false) { return 2 * half + (bf ? 48 : 34); }
// LDS bytes of the matrix-core adjoint: the staged window and the zero-padded filter table,
// both in the operand type
__host__ __device__ inline int64_t ma_lds(int half, int C, int es, bool bf) {
  return (int64_t)C * (16 * ma_ws(half, bf) + ma_fl(half, bf)) * (bf ? 2 : es);
}

// One g position (C values, re then im) through a buffer resource; 0 outside its range.
template <typename T, int C>
__device__ inline void ma_load(__amdgpu_buffer_rsrc_t r, int off, T (&v)[C]) {
  if constexpr (sizeof(T) * C == 4) {
    const unsigned u = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    __builtin_memcpy(v, &u, 4);
  } else if constexpr (sizeof(T) * C == 8) {
    const auto u = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    __builtin_memcpy(v, &u, 8);
  } else {
    const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    __builtin_memcpy(v, &u, 16);
  }
}

template <typename T, bool CPLX, int D, bool BF>  // BF: bf16 operands (T = float)
__global__ void __launch_bounds__(NT) morlet_adjoint_mfma_kernel(Stage st, const T* __restrict__ g,
                                                                 T* __restrict__ gx, int g_scales,
                                                                 int64_t rows, int rblocks,
                                                                 int itiles, int64_t lo,
                                                                 int64_t hi, int accumulate) {
  constexpr int C = CPLX ? 2 : 1;
  constexpr int RW = 16 / D;            // rows of a workgroup
  constexpr int LD = __builtin_ctz(D);
  static_assert(MA_PFN % D == 0 && MA_PFN / D == RW, "D * MA_WL slots per row");
  static_assert(!BF || std::is_same<T, float>::value, "bf16 operands with float storage");
  typedef typename Mfma16<T>::v4 v4;
  typedef typename std::conditional<BF, uint16_t, T>::type E;  // staged window element
  typedef short v4s __attribute__((ext_vector_type(4)));
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int half = st.half, dil = st.dil;
  const int WS = ma_ws(half, BF), FL = ma_fl(half, BF), PADL = half + 15;
  E* const U = reinterpret_cast<E*>(smem_raw);  // [C][16][WS]
  E* const Fz = U + C * 16 * WS;                // [C][FL]: F_{s,c}[z - PADL], 0 elsewhere
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t blk = blockIdx.x;
  const int rb = (int)(blk % rblocks);
  const int64_t rest = blk / rblocks;
  const int it = (int)(rest % itiles);
  const int64_t row0 = (rest / itiles) * RW;
  const int rho0 = rb * D;
  const int64_t i0 = (int64_t)it * MA_TI;
  const T* taps = static_cast<const T*>(st.taps);

  if (!accumulate) {  // zero the positions g does not reach, spread over the row group's blocks
    const int64_t outside = lo + (st.n_in - hi);
    const int64_t nb = (int64_t)itiles * rblocks, b = (int64_t)it * rblocks + rb;
    for (int64_t e = b * NT + tid; e < RW * outside; e += nb * NT) {
      const int64_t r = row0 + e / outside, j = e % outside;
      if (r < rows) gx[r * st.n_in + (j < lo ? j : hi + (j - lo))] = T(0);
    }
  }

  // staging slots: load m of a thread covers row m >> LD, flat index f = tid + NT (m & (D-1))
  // of the row's D * MA_WL slots, i.e. window position j = f >> LD of residue rho0 + (f & (D-1))
  auto plane = [&](int r, int s) {
    const int64_t row = row0 + r;
    const bool ok = row < rows;
    const T* base = ok ? g + ((row * g_scales + st.chan[s]) * st.n_out) * C : g;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), (short)0,
                                             ok ? (int)(st.n_out * C * (int64_t)sizeof(T)) : 0,
                                             0x00020000);
  };
  T pf[MA_PFN][C];
  auto prefetch = [&](int s) {
    const int64_t qb = lo - st.x_off + rho0 + (int64_t)dil * (i0 - st.sup[s]);
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const __amdgpu_buffer_rsrc_t pr = plane(r, s);
#pragma unroll
      for (int m = 0; m < D; ++m) {
        const int f = tid + NT * m;
        const int64_t q = qb + (f & (D - 1)) + (int64_t)dil * (f >> LD);
        ma_load<T, C>(pr, (int)(q * C * (int64_t)sizeof(T)), pf[r * D + m]);
      }
    }
  };
  const int i_l = lane & 15, kap = lane >> 4;
  v4 acc[MA_NB];
#pragma unroll
  for (int b = 0; b < MA_NB; ++b) acc[b] = v4{T(0), T(0), T(0), T(0)};
  if (st.n_scales > 0) prefetch(0);
  for (int s = 0; s < st.n_scales; ++s) {
    const int sup = st.sup[s];
    const int wl = MA_TI + 2 * sup + ma_ext(BF);  // staged window positions
    const T* tp = taps + s * (half + 1) * C;
    // F_{s,c}[k], |k| <= sup, from the compact taps (0 beyond the support)
    auto filt = [&](int c, int k) {
      const int a = k < 0 ? -k : k;
      T v = T(0);
      if (a <= sup) {
        v = tp[a * C + c];
        if (c == 1) v = k > 0 ? v : (k < 0 ? -v : T(0));
      }
      return v;
    };
    __syncthreads();  // the previous scale's reads of U and the filter table are done
#pragma unroll
    for (int r = 0; r < RW; ++r) {
#pragma unroll
      for (int m = 0; m < D; ++m) {
        const int f = tid + NT * m, j = f >> LD;
        if (j < wl) {
          E* u = U + (r * D + (f & (D - 1))) * WS + j;
#pragma unroll
          for (int c = 0; c < C; ++c) {
            if constexpr (BF) u[c * 16 * WS] = f2bf(pf[r * D + m][c]);
            else u[c * 16 * WS] = pf[r * D + m][c];
          }
        }
      }
    }
    const int steps = BF ? (16 + 2 * sup + 15) / 16 : (16 + 2 * sup + 3) / 4;
    for (int e = tid; e < C * FL; e += NT) {
      const T v = filt(e / FL, e % FL - PADL);
      if constexpr (BF) Fz[e] = f2bf(v);
      else Fz[e] = v;
    }
    __syncthreads();
    if (s + 1 < st.n_scales) prefetch(s + 1);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if constexpr (BF) {
        // A: U[l % 16][16 tb + 16 t + 4 (l / 16) + v], v < 4 (8-byte aligned: WS % 4 == 0);
        // B: Z[16 t + 4 (l / 16) + v][l % 16] = F[16 t + 4 (l / 16) + v - l % 16 - sup]
        const E* ua = U + (c * 16 + i_l) * WS + 16 * MA_NB * wave + 4 * kap;
        const E* zb = Fz + c * FL + PADL + 4 * kap - i_l - sup;
        for (int t = 0; t < steps; ++t) {
          v4s b;
#pragma unroll
          for (int v = 0; v < 4; ++v) b[v] = (short)zb[16 * t + v];
#pragma unroll
          for (int bb = 0; bb < MA_NB; ++bb) {
            const v4s a = *reinterpret_cast<const v4s*>(ua + 16 * bb + 16 * t);
            acc[bb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc[bb], 0, 0, 0);
          }
        }
      } else {
        const E* ua = U + (c * 16 + i_l) * WS + 16 * MA_NB * wave + kap;
        const T* zb = Fz + c * FL + PADL + kap - i_l - sup;
        for (int t = 0; t < steps; ++t) {
          const T b = zb[4 * t];
#pragma unroll
          for (int bb = 0; bb < MA_NB; ++bb)
            acc[bb] = Mfma16<T>::mma(ua[16 * bb + 4 * t], b, acc[bb]);
        }
      }
    }
  }
  // result element e of lane l: line Mfma16::row(l, e) = (row, residue), output i = l % 16
#pragma unroll
  for (int bb = 0; bb < MA_NB; ++bb) {
    const int64_t i = i0 + 16 * (MA_NB * wave + bb) + i_l;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int mline = Mfma16<T>::row(lane, e);
      const int64_t r = row0 + (mline >> LD);
      const int64_t p = lo + rho0 + (mline & (D - 1)) + (int64_t)dil * i;
      if (p < hi && r < rows) {
        T* o = gx + r * st.n_in + p;
        *o = accumulate ? *o + acc[bb][e] : acc[bb][e];
      }
    }
  }
}

// ------------------------------------------------------------------ half-band chain step
// y[n] (+)= t0 x[n + b] + sum_{t odd <= c} taps[t] (x[n + b - dil t] + x[n + b + dil t])
template <typename T>
__global__ void __launch_bounds__(NT) halfband_kernel(const T* __restrict__ x,
                                                      const T* __restrict__ taps,
                                                      T* __restrict__ y, int64_t n_in,
                                                      int64_t n_out, int c, int64_t b, int dil,
                                                      int tiles, int accumulate) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* X = reinterpret_cast<T*>(smem_raw);
  const int64_t row = blockIdx.x / tiles;
  const int64_t n0 = (int64_t)(blockIdx.x % tiles) * TT;
  const int span = TT + 2 * dil * c;
  stage_row(X, x + row * n_in, n0 + b - (int64_t)dil * c, span, n_in);
  __syncthreads();
  const int tid = threadIdx.x;
  const int base = tid + dil * c;
  T acc[V];
  const T t0 = taps[0];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = t0 * X[base + NT * v];
  for (int t = 1; t <= c; t += 2) {
    const T h = taps[t];
#pragma unroll
    for (int v = 0; v < V; ++v)
      acc[v] = fma(h, X[base + NT * v - dil * t] + X[base + NT * v + dil * t], acc[v]);
  }
  T* yrow = y + row * n_out;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t n = n0 + tid + NT * v;
    if (n < n_out) yrow[n] = accumulate ? yrow[n] + acc[v] : acc[v];
  }
}

// ------------------------------------------------------------------ fused mix
// forward:  y[r, n] (+)= sum_s a[d, chan_s] |W_s| + b[d, chan_s] Re W_s,  d = (r + row0) % D
// backward: gw[r, s, n] = gy (a Re W / |W| + b,  a Im W / |W|)  (|W| = 0 -> 0), and per
//           workgroup partial sums (sum gy |W|, sum gy Re W) per local scale.
template <typename T, bool CPLX, bool GRAD>
__global__ void __launch_bounds__(NT) mix_kernel(Stage st, const T* __restrict__ a,
                                                 const T* __restrict__ b, int s_total_w, int D,
                                                 int64_t row0, T* __restrict__ y,
                                                 const T* __restrict__ gy, T* __restrict__ gw,
                                                 T* __restrict__ partial, int tiles,
                                                 int accumulate) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  constexpr int C = CPLX ? 2 : 1;
  T* X = reinterpret_cast<T*>(smem_raw);
  const int half = st.half, dil = st.dil;
  const int span = TT + 2 * dil * half;
  T* red = X + ((span + 3) & ~3);  // NT / 64 waves x 2 partial sums
  const int64_t row = blockIdx.x / tiles;
  const int64_t n0 = (int64_t)(blockIdx.x % tiles) * TT;
  const int tid = threadIdx.x;
  stage_row(X, static_cast<const T*>(st.x) + row * st.n_in, n0 + st.x_off - (int64_t)dil * half,
            span, st.n_in);
  __syncthreads();
  const int d = (int)((row + row0) % D);
  const T* taps = static_cast<const T*>(st.taps);
  T gyv[V], out[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t n = n0 + tid + NT * v;
    out[v] = T(0);
    gyv[v] = (GRAD && n < st.n_out) ? gy[row * st.n_out + n] : T(0);
  }
  for (int s0 = 0; s0 < st.n_scales; s0 += SG) {
    const int ns = min(SG, st.n_scales - s0);
    T re[V][SG], im[V][SG];
    bank_group<T, CPLX>(X, taps, half, dil, s0, ns, st.sup[s0 + ns - 1], re, im);
#pragma unroll
    for (int s = 0; s < SG; ++s) {
      if (s >= ns) break;
      const int gs = st.chan[s0 + s];
      const T av = a[d * s_total_w + gs];
      const T bv = b[d * s_total_w + gs];
      T sa = T(0), sb = T(0);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int64_t n = n0 + tid + NT * v;
        const T rv = re[v][s], iv = im[v][s];
        T mag = fabs(rv), inv = T(0);
        if (CPLX) {
          if (GRAD) mag_inv(fma(rv, rv, iv * iv), mag, inv);
          else mag = hw_sqrt(fma(rv, rv, iv * iv));
        } else if (GRAD) {
          inv = mag > T(0) ? T(1) / mag : T(0);  // rv inv = sign of Re W
        }
        if (!GRAD) {
          out[v] = fma(av, mag, fma(bv, rv, out[v]));
        } else if (n < st.n_out) {
          T* gwp = gw + ((row * st.n_scales + s0 + s) * st.n_out + n) * C;
          if (CPLX) {
            typedef T v2 __attribute__((ext_vector_type(2)));
            *reinterpret_cast<v2*>(gwp) = v2{gyv[v] * (av * rv * inv + bv), gyv[v] * (av * iv * inv)};
          } else {
            // real transform: |W| = |Re W|, d|W|/dRe W = sign
            gwp[0] = gyv[v] * (av * rv * inv + bv);
          }
          sa = fma(gyv[v], mag, sa);
          sb = fma(gyv[v], rv, sb);
        }
      }
      if (GRAD) {
        // workgroup sum of (sa, sb): wave reduction, then across the NT / 64 waves
        for (int o = 32; o > 0; o >>= 1) {
          sa += __shfl_xor(sa, o);
          sb += __shfl_xor(sb, o);
        }
        __syncthreads();
        if ((tid & 63) == 0) {
          red[2 * (tid >> 6)] = sa;
          red[2 * (tid >> 6) + 1] = sb;
        }
        __syncthreads();
        if (tid == 0) {
          T ta = T(0), tb = T(0);
          for (int w = 0; w < NT / 64; ++w) {
            ta += red[2 * w];
            tb += red[2 * w + 1];
          }
          T* pp = partial + ((int64_t)blockIdx.x * st.n_scales + s0 + s) * 2;
          pp[0] = ta;
          pp[1] = tb;
        }
      }
    }
  }
  if (!GRAD) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int64_t n = n0 + tid + NT * v;
      if (n < st.n_out) {
        T* yp = y + row * st.n_out + n;
        *yp = accumulate ? *yp + out[v] : out[v];
      }
    }
  }
}

// ------------------------------------------------------------------ spectral softmax
// V values: per channel (v_pos = 0): V[(r + row0) % nch][chan_s]   (layout (nch, S_total))
//           per position (v_pos = 1): V[(r + row0) / nch][chan_s][n] (layout (G, S_total, N))
struct SoftArgs {
  const void* v;
  int64_t s_total;
  int32_t nch;
  int32_t v_pos;
  int64_t row0;
  double inv_tau;
};

// The V row of a workgroup's signal row (the division by nch once per workgroup, not per
// scale and position): per channel, V[(r % nch)][.]; per position, the (S_total, N) plane of
// group r / nch.
template <typename T>
__device__ inline const T* v_row(const SoftArgs& sa, const T* V, int64_t row, int64_t n_out) {
  const int64_t r = row + sa.row0;
  return sa.v_pos ? V + (r / sa.nch) * sa.s_total * n_out : V + (r % sa.nch) * sa.s_total;
}
template <typename T>
__device__ inline T v_value(const SoftArgs& sa, const T* vrow, int gs, int64_t n, int64_t n_out) {
  return sa.v_pos ? vrow[gs * n_out + n] : vrow[gs];
}

// forward: fold the stage into the online softmax state (m, l, num) of every position;
// first: no state yet (m = -inf, l = 0, num = 0); last: write out = num / l into `num`.
template <typename T>
__global__ void __launch_bounds__(NT) softmax_forward_kernel(Stage st, SoftArgs sa,
                                                             T* __restrict__ m, T* __restrict__ l,
                                                             T* __restrict__ num, int tiles,
                                                             int first, int last) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* X = reinterpret_cast<T*>(smem_raw);
  const int half = st.half, dil = st.dil;
  const int span = TT + 2 * dil * half;
  const int64_t row = blockIdx.x / tiles;
  const int64_t n0 = (int64_t)(blockIdx.x % tiles) * TT;
  const int tid = threadIdx.x;
  stage_row(X, static_cast<const T*>(st.x) + row * st.n_in, n0 + st.x_off - (int64_t)dil * half,
            span, st.n_in);
  __syncthreads();
  const T* vrow = v_row(sa, static_cast<const T*>(sa.v), row, st.n_out);
  constexpr T kLog = SoftExp<T>::kLog;
  const T kt = T(sa.inv_tau) * kLog;  // |W| -> |W| / tau in the exponential's base
  T mm[V], ll[V], nn[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t n = n0 + tid + NT * v;
    const int64_t idx = row * st.n_out + min(n, st.n_out - 1);
    mm[v] = first ? -INFINITY : m[idx] * kLog;
    ll[v] = first ? T(0) : l[idx];
    nn[v] = first ? T(0) : num[idx];
  }
  const T* taps = static_cast<const T*>(st.taps);
  for (int s0 = 0; s0 < st.n_scales; s0 += SG) {
    const int ns = min(SG, st.n_scales - s0);
    T re[V][SG], im[V][SG];
    bank_group<T, true>(X, taps, half, dil, s0, ns, st.sup[s0 + ns - 1], re, im);
#pragma unroll
    for (int s = 0; s < SG; ++s) {
      if (s >= ns) break;
      const int gs = st.chan[s0 + s];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int64_t n = min(n0 + tid + NT * v, st.n_out - 1);
        const T av = hw_sqrt(fma(re[v][s], re[v][s], im[v][s] * im[v][s])) * kt;
        const T val = v_value(sa, vrow, gs, n, st.n_out);
        // one exponential per value: exp(-|av - m|) rescales the state when av is the new
        // maximum and weighs av otherwise (first frequency: m = -inf, exp(-inf) = 0)
        const T dd = av - mm[v];
        const T ex = SoftExp<T>::ex(-fabs(dd));
        const bool up = dd > T(0);
        const T sc = up ? ex : T(1), e = up ? T(1) : ex;
        ll[v] = fma(ll[v], sc, e);
        nn[v] = fma(nn[v], sc, e * val);
        mm[v] = up ? av : mm[v];
      }
    }
  }
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t n = n0 + tid + NT * v;
    if (n < st.n_out) {
      const int64_t idx = row * st.n_out + n;
      m[idx] = mm[v] * (T(1) / kLog);
      l[idx] = ll[v];
      num[idx] = last ? nn[v] / ll[v] : nn[v];
    }
  }
}

// backward: p = exp(|W|/tau - m) / l, gp = gy p;  gw = gp (V - out) / tau * W / |W|;
// dL/dV partials: per channel, per workgroup and local scale sum_n gp (partial (blocks, S_j));
// per position, gp itself (partial (rows, S_j, n_out)), reduced over channels afterwards.
template <typename T>
__global__ void __launch_bounds__(NT) softmax_backward_kernel(Stage st, SoftArgs sa,
                                                              const T* __restrict__ m,
                                                              const T* __restrict__ l,
                                                              const T* __restrict__ out,
                                                              const T* __restrict__ gy,
                                                              T* __restrict__ gw,
                                                              T* __restrict__ partial,
                                                              int tiles) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* X = reinterpret_cast<T*>(smem_raw);
  const int half = st.half, dil = st.dil;
  const int span = TT + 2 * dil * half;
  T* red = X + ((span + 3) & ~3);
  const int64_t row = blockIdx.x / tiles;
  const int64_t n0 = (int64_t)(blockIdx.x % tiles) * TT;
  const int tid = threadIdx.x;
  stage_row(X, static_cast<const T*>(st.x) + row * st.n_in, n0 + st.x_off - (int64_t)dil * half,
            span, st.n_in);
  __syncthreads();
  const T* vrow = v_row(sa, static_cast<const T*>(sa.v), row, st.n_out);
  const T inv_tau = T(sa.inv_tau);
  constexpr T kLog = SoftExp<T>::kLog;
  const T kt = inv_tau * kLog;
  T mm[V], il[V], oo[V], gg[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t n = n0 + tid + NT * v;
    const int64_t idx = row * st.n_out + min(n, st.n_out - 1);
    const bool ok = n < st.n_out;
    mm[v] = m[idx] * kLog;
    il[v] = T(1) / l[idx];
    oo[v] = out[idx];
    gg[v] = ok ? gy[idx] : T(0);
  }
  const T* taps = static_cast<const T*>(st.taps);
  for (int s0 = 0; s0 < st.n_scales; s0 += SG) {
    const int ns = min(SG, st.n_scales - s0);
    T re[V][SG], im[V][SG];
    bank_group<T, true>(X, taps, half, dil, s0, ns, st.sup[s0 + ns - 1], re, im);
#pragma unroll
    for (int s = 0; s < SG; ++s) {
      if (s >= ns) break;
      const int gs = st.chan[s0 + s];
      T sv = T(0);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int64_t n = n0 + tid + NT * v;
        const bool ok = n < st.n_out;
        const int64_t nc = min(n, st.n_out - 1);
        const T rv = re[v][s], iv = im[v][s];
        T mag, inv;
        mag_inv(fma(rv, rv, iv * iv), mag, inv);
        const T p = SoftExp<T>::ex(fma(mag, kt, -mm[v])) * il[v];
        const T gp = ok ? gg[v] * p : T(0);
        const T val = v_value(sa, vrow, gs, nc, st.n_out);
        const T coef = gp * (val - oo[v]) * inv_tau * inv;
        if (ok) {
          typedef T v2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<v2*>(gw + ((row * st.n_scales + s0 + s) * st.n_out + n) * 2) =
              v2{coef * rv, coef * iv};
          if (sa.v_pos) partial[(row * st.n_scales + s0 + s) * st.n_out + n] = gp;
        }
        sv += gp;
      }
      if (!sa.v_pos) {
        for (int o = 32; o > 0; o >>= 1) sv += __shfl_xor(sv, o);
        __syncthreads();
        if ((tid & 63) == 0) red[tid >> 6] = sv;
        __syncthreads();
        if (tid == 0) {
          T tsum = T(0);
          for (int w = 0; w < NT / 64; ++w) tsum += red[w];
          partial[(int64_t)blockIdx.x * st.n_scales + s0 + s] = tsum;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ deterministic reductions
// out[o] (+)= sum_{i < count} in[o * count + i]: one workgroup per output, fixed order
// (per-thread strided sums, then a fixed shuffle / LDS tree).
template <typename T>
__global__ void __launch_bounds__(NT) reduce_cols_kernel(const T* __restrict__ in,
                                                         T* __restrict__ out, int64_t count,
                                                         int accumulate) {
  __shared__ T red[NT / 64];
  const int64_t o = blockIdx.x;
  const T* p = in + o * count;
  T acc = T(0);
  for (int64_t i = threadIdx.x; i < count; i += NT) acc += p[i];
  for (int d = 32; d > 0; d >>= 1) acc += __shfl_xor(acc, d);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    T t = T(0);
    for (int w = 0; w < NT / 64; ++w) t += red[w];
    out[o] = accumulate ? out[o] + t : t;
  }
}

// dL/dV of the per-position spectral softmax: the backward's partials (groups nch rows,
// n_scales, n_out) summed over each group's nch rows in row order (deterministic) and added to
// the V gradient at the scales' global indices: grid (groups * n_scales, tiles of NT
// positions), one position per thread, the rows' loads unrolled so several are in flight.
struct DvArgs {
  int32_t chan[MAXS];
};
template <typename T>
__global__ void __launch_bounds__(NT) softmax_dv_kernel(const T* __restrict__ part,
                                                        T* __restrict__ gv, DvArgs ca, int nch,
                                                        int n_scales, int64_t v_s_total,
                                                        int64_t n_out, int64_t g0, int tiles) {
  const int64_t gs = blockIdx.x / tiles;  // (group, local scale)
  const int64_t g = gs / n_scales;
  const int s = (int)(gs % n_scales);
  const int64_t n = (int64_t)(blockIdx.x % tiles) * NT + threadIdx.x;
  if (n >= n_out) return;
  const T* src = part + (g * nch * n_scales + s) * n_out + n;  // row c at c n_scales n_out
  const int64_t rstride = (int64_t)n_scales * n_out;
  T acc = T(0);
#pragma unroll 8
  for (int c = 0; c < nch; ++c) acc += src[c * rstride];
  gv[((g0 + g) * v_s_total + ca.chan[s]) * n_out + n] += acc;
}

// ------------------------------------------------------------------ filter synthesis
// Sampled Morlet filters (reference cwt.py:181-203): row i C + ch, column center + k,
//   t = k dil_i / s_i,  env = exp(-t^2 / 2) [|k| <= sup_i],  amp = pi^(-1/4) dil_i / s_i^p,
//   re = (cos(w0 t) - exp(-w0^2 / 2)) env amp,   im = sin(w0 t) env amp,
// with p = 1/2 (l2 norm) or 1 (l1).  Every value is computed at a = |k| in float64 and
// written to both sides, so real rows are exactly even and imaginary rows exactly odd (the
// bank kernels above rely on that).  The gradient kernel applies the derivatives
//   s d re/ds  = env amp [w0 t sin(w0 t) + (cos(w0 t) - e)(t^2 - p)],     e = exp(-w0^2 / 2)
//   s d im/ds  = env amp [sin(w0 t)(t^2 - p) - w0 t cos(w0 t)]
//   d re/dw0   = env amp [w0 e - t sin(w0 t)],   d im/dw0 = env amp t cos(w0 t)
// to the pair sums gH[c + a] + gH[c - a] (real rows) and differences gH[c + a] - gH[c - a]
// (imaginary rows); one wave reduces one scale, so the result is deterministic.
constexpr int MAXF = FDWT_MORLET_MAX_FILTERS;
constexpr double PI_M14 = 0.75112554446494248286;  // pi^(-1/4)

struct FilterArgs {
  const double* scales;  // (n_scales) device
  const double* w0;      // (1) device
  int32_t n_scales, center, C, l2;
  int32_t dil[MAXF];
  int32_t sup[MAXF];
};

// The per-scale tables are indexed per lane, so they are read in place from the kernel
// argument segment (a by-value copy indexed at run time would go to scratch).
#if defined(__HIP_DEVICE_COMPILE__)
#define FDWT_FILTER_ARGS(name)                                              \
  typedef __attribute__((address_space(4))) const FilterArgs FArgs_;         \
  FArgs_& name = *(FArgs_*)__builtin_amdgcn_kernarg_segment_ptr()
#else  // the host pass only type-checks kernel bodies
#define FDWT_FILTER_ARGS(name) const FilterArgs name {}
#endif

struct MorletSample {
  double t, env_amp, c, sn;  // t, env * amp, cos(w0 t), sin(w0 t)
};

__device__ inline MorletSample morlet_sample(double s, double w0, int dil, int sup, int l2,
                                             int a) {
  MorletSample m;
  m.t = (double)a * (double)dil / s;
  const double env = a <= sup ? exp(-0.5 * m.t * m.t) : 0.0;
  m.env_amp = env * (PI_M14 * (double)dil / (l2 ? sqrt(s) : s));
  sincos(w0 * m.t, &m.sn, &m.c);
  return m;
}

template <typename T>
__global__ void __launch_bounds__(NT) morlet_filters_kernel(FilterArgs, T* __restrict__ H) {
  FDWT_FILTER_ARGS(fa);
  const int w = fa.center + 1;
  const int64_t e = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (e >= (int64_t)fa.n_scales * w) return;
  const int i = (int)(e / w), a = (int)(e % w);
  const double w0 = fa.w0[0];
  const MorletSample m = morlet_sample(fa.scales[i], w0, fa.dil[i], fa.sup[i], fa.l2, a);
  const double re = (m.c - exp(-0.5 * w0 * w0)) * m.env_amp;
  const int W = 2 * fa.center + 1;
  T* row = H + (int64_t)i * fa.C * W + fa.center;
  row[a] = T(re);
  row[-a] = T(re);
  if (fa.C == 2) {
    const double im = m.sn * m.env_amp;
    row[W + a] = T(im);
    if (a > 0) row[W - a] = T(-im);
  }
}

template <typename T>
__global__ void __launch_bounds__(NT) morlet_filters_backward_kernel(FilterArgs,
                                                                     const T* __restrict__ gH,
                                                                     double* __restrict__ g_scales,
                                                                     double* __restrict__ g_w0) {
  FDWT_FILTER_ARGS(fa);
  __shared__ double w0_part[NT / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int W = 2 * fa.center + 1;
  const double w0 = fa.w0[0];
  const double ew = exp(-0.5 * w0 * w0);
  const double p = fa.l2 ? 0.5 : 1.0;
  double gw = 0.0;
  for (int i = wave; i < fa.n_scales; i += NT / 64) {
    const double s = fa.scales[i];
    const T* row = gH + (int64_t)i * fa.C * W + fa.center;
    double gs = 0.0;
    for (int a = lane; a <= fa.center; a += 64) {
      const MorletSample m = morlet_sample(s, w0, fa.dil[i], fa.sup[i], fa.l2, a);
      const double gr = a ? (double)row[a] + (double)row[-a] : (double)row[0];
      const double tt = m.t * m.t - p;
      gs += gr * m.env_amp * (w0 * m.t * m.sn + (m.c - ew) * tt);
      gw += gr * m.env_amp * (w0 * ew - m.t * m.sn);
      if (fa.C == 2 && a > 0) {
        const double gi = (double)row[W + a] - (double)row[W - a];
        gs += gi * m.env_amp * (m.sn * tt - w0 * m.t * m.c);
        gw += gi * m.env_amp * m.t * m.c;
      }
    }
    for (int d = 32; d > 0; d >>= 1) gs += __shfl_xor(gs, d);
    if (lane == 0) g_scales[i] = gs / s;
  }
  for (int d = 32; d > 0; d >>= 1) gw += __shfl_xor(gw, d);
  if (lane == 0) w0_part[wave] = gw;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int v = 0; v < NT / 64; ++v) t += w0_part[v];
    g_w0[0] = t;
  }
}

// ------------------------------------------------------------------ host helpers
int fill_stage(Stage& st, const void* x, const void* taps, int64_t n_in, int64_t n_out,
               int64_t x_off, int32_t n_scales, int32_t half, const int32_t* support,
               const int32_t* chan, int32_t dil, int32_t channels) {
  if (!x || !taps || n_in < 0 || n_out < 0 || n_scales < 1 || n_scales > MAXS || half < 0 ||
      dil < 1 || !support || !chan || (channels != 1 && channels != 2))
    return FDWT_ERR_ARG;
  if ((int64_t)dil * half > (1 << 20)) return FDWT_ERR_TOO_LONG;
  st.x = x;
  st.taps = taps;
  st.n_in = n_in;
  st.n_out = n_out;
  st.x_off = x_off;
  st.n_scales = n_scales;
  st.half = half;
  st.dil = dil;
  st.C = channels;
  for (int s = 0; s < n_scales; ++s) {
    if (support[s] < 0 || support[s] > half || chan[s] < 0) return FDWT_ERR_ARG;
    if (s > 0 && support[s] < support[s - 1]) return FDWT_ERR_ARG;  // sorted by support
    st.sup[s] = support[s];
    st.chan[s] = chan[s];
  }
  return 0;
}

inline size_t tile_lds(const Stage& st, int cs, int extra_elems) {
  const int64_t span = TT + 2 * (int64_t)st.dil * st.half;
  return (size_t)(((span + 3) & ~3) + extra_elems) * cs;
}

template <typename K>
inline bool allow_full_lds(K kernel) {
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return true;
}

// Workgroups of `kernel` (NT threads, `lds` bytes) resident on the whole device at once,
// at most `cap` (a persistent grid: one round of workgroups).
template <typename K>
inline int resident_blocks(K kernel, size_t lds, int64_t cap) {
  int dev = 0, per_cu = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel),
                                                   NT, lds) != hipSuccess)
    per_cu = 1, cus = 256;
  const int64_t n = (int64_t)std::max(per_cu, 1) * std::max(cus, 1);
  return (int)std::max<int64_t>(1, std::min(n, cap));
}

template <typename K, typename... Args>
int launch(K kernel, int64_t blocks, size_t lds, hipStream_t st, Args... args) {
  if (blocks <= 0) return 0;
  if (blocks > (int64_t)(0xffffffffu / NT)) return FDWT_ERR_ARG;  // 2^32 - 1 threads per launch
  if (lds > 160 * 1024) return FDWT_ERR_TOO_LONG;
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(NT), lds, st, args...);
  FDWT_CHECK_LAUNCH();
  return 0;
}

}  // namespace
}  // namespace fdwt

using namespace fdwt;

#define FDWT_LDS_ONCE(K)                                   \
  do {                                                     \
    static const bool lds_ok_ = allow_full_lds(K);         \
    (void)lds_ok_;                                         \
  } while (0)

extern "C" int fdwt_halfband(const void* x, const void* taps, void* y, int64_t rows,
                             int64_t n_in, int64_t n_out, int32_t c, int64_t b, int32_t dil,
                             int32_t accumulate, int32_t dtype, void* stream) {
  if (!x || !taps || !y || rows < 0 || n_in < 1 || n_out < 0 || c < 0 || dil < 1 ||
      (dtype != FDWT_F32 && dtype != FDWT_F64))
    return FDWT_ERR_ARG;
  if (rows == 0 || n_out == 0) return 0;
  const int tiles = (int)cdiv(n_out, TT);
  const int64_t span = TT + 2 * (int64_t)dil * c;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FDWT_F32) {
    auto k = halfband_kernel<float>;
    FDWT_LDS_ONCE(k);
    return launch(k, rows * tiles, (size_t)span * 4, st, (const float*)x, (const float*)taps,
                  (float*)y, n_in, n_out, c, b, dil, tiles, accumulate);
  }
  auto k = halfband_kernel<double>;
  FDWT_LDS_ONCE(k);
  return launch(k, rows * tiles, (size_t)span * 8, st, (const double*)x, (const double*)taps,
                (double*)y, n_in, n_out, c, b, dil, tiles, accumulate);
}

extern "C" int fdwt_morlet_forward(const void* x, const void* taps, void* y, int64_t rows,
                                   int64_t n_in, int64_t n_out, int64_t x_off, int32_t n_scales,
                                   int32_t half, const int32_t* support, const int32_t* chan,
                                   int32_t dil, int32_t channels, int32_t s_total, int32_t dtype,
                                   void* stream) {
  Stage st;
  int e = fill_stage(st, x, taps, n_in, n_out, x_off, n_scales, half, support, chan, dil, channels);
  if (e) return e;
  if (!y || rows < 0 || s_total < n_scales || (dtype != FDWT_F32 && dtype != FDWT_F64))
    return FDWT_ERR_ARG;
  for (int s = 0; s < n_scales; ++s)
    if (chan[s] >= s_total) return FDWT_ERR_ARG;
  if (rows == 0 || n_out == 0) return 0;
  if (n_in < 1) return FDWT_ERR_ARG;  // x is staged: a row needs a sample
  const int tiles = (int)cdiv(n_out, TT);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const int cs = dtype == FDWT_F64 ? 8 : 4;
  const size_t lds = tile_lds(st, cs, 0);
#define FWD(TYPE, CPLX)                                                                  \
  do {                                                                                   \
    auto k = morlet_forward_kernel<TYPE, CPLX>;                                          \
    FDWT_LDS_ONCE(k);                                                                    \
    return launch(k, rows * tiles, lds, hs, st, (TYPE*)y, (int)s_total, tiles);          \
  } while (0)
  if (dtype == FDWT_F32) {
    if (channels == 2) FWD(float, true);
    FWD(float, false);
  }
  if (channels == 2) FWD(double, true);
  FWD(double, false);
#undef FWD
}

extern "C" int fdwt_morlet_backward_x(const void* g, const void* taps, void* gx, int64_t rows,
                                      int64_t n_in, int64_t n_out, int64_t x_off,
                                      int32_t n_scales, int32_t half, const int32_t* support,
                                      const int32_t* chan, int32_t dil, int32_t channels,
                                      int32_t g_scales, int32_t accumulate, int32_t dtype,
                                      void* stream) {
  Stage st;
  // the stage's x is unused here; pass g to satisfy the null check
  int e = fill_stage(st, g, taps, n_in, n_out, x_off, n_scales, half, support, chan, dil, channels);
  if (e) return e;
  if (!gx || rows < 0 || g_scales < 1 ||
      (dtype != FDWT_F32 && dtype != FDWT_F64 && dtype != FDWT_F32_BF16))
    return FDWT_ERR_ARG;
  for (int s = 0; s < n_scales; ++s)
    if (chan[s] >= g_scales) return FDWT_ERR_ARG;
  if (rows == 0 || n_in == 0) return 0;
  if (n_out == 0) return FDWT_ERR_ARG;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const int cs = dtype == FDWT_F64 ? 8 : 4;
  {
    // matrix-core kernel over the range g reaches (as the windowed kernel below), when its
    // LDS (the staged window of 16 rows and the filter tables) fits and every g position a
    // workgroup touches (-dil (half + MA_TI + 4) .. n_out + the same) is within the 2^31
    // bytes of a plane's 32-bit buffer offsets
    const int64_t reach = (int64_t)dil * half;
    const int64_t lo = std::min(std::max(x_off - reach, (int64_t)0), n_in);
    const int64_t hi = std::min(std::max(x_off + n_out + reach, lo), n_in);
    const bool bf = dtype == FDWT_F32_BF16;
    const size_t lds = (size_t)ma_lds(half, channels, cs, bf);
    const int64_t itiles = cdiv(std::max((int64_t)1, cdiv(hi - lo, dil)), MA_TI);
    const int d = dil < 16 ? dil : 16;  // residues per workgroup line group
    const int64_t rblocks = dil / d;
    const int64_t blocks = cdiv(rows, 16 / d) * itiles * rblocks;
    if ((dil & (dil - 1)) == 0 && MA_TI + 2 * half + ma_ext(bf) <= MA_WL && lds <= 64 * 1024 &&
        itiles <= INT32_MAX &&
        (n_out + 2 * (int64_t)dil * (half + MA_TI + 16)) * channels * cs < ((int64_t)1 << 31)) {
#define ADM_D(TYPE, CPLX, DD, BF)                                                            \
  case DD: {                                                                                 \
    auto k = morlet_adjoint_mfma_kernel<TYPE, CPLX, DD, BF>;                                 \
    FDWT_LDS_ONCE(k);                                                                        \
    return launch(k, blocks, lds, hs, st, (const TYPE*)g, (TYPE*)gx, (int)g_scales, rows,     \
                  (int)rblocks, (int)itiles, lo, hi, (int)accumulate);                       \
  }
#define ADM(TYPE, CPLX, BF)                                                                  \
  switch (d) {                                                                               \
    ADM_D(TYPE, CPLX, 1, BF) ADM_D(TYPE, CPLX, 2, BF) ADM_D(TYPE, CPLX, 4, BF)               \
    ADM_D(TYPE, CPLX, 8, BF) ADM_D(TYPE, CPLX, 16, BF) default: break;                       \
  }
      if (bf) {
        if (channels == 2) ADM(float, true, true) else ADM(float, false, true)
      } else if (dtype == FDWT_F32) {
        if (channels == 2) ADM(float, true, false) else ADM(float, false, false)
      } else {
        if (channels == 2) ADM(double, true, false) else ADM(double, false, false)
      }
#undef ADM
#undef ADM_D
    }
    if (bf) dtype = FDWT_F32;  // bf16 operands are a permission: the other kernels stay fp32
  }
  if ((dil & (dil - 1)) == 0 &&
      (n_out + 2 * (int64_t)dil * (half + RUN + 1)) * channels * cs < ((int64_t)1 << 31)) {
    // windowed kernel (power-of-two dilation, and g positions -2 dil H .. n_out + 2 dil H of
    // a plane within the 2^31 bytes of its 32-bit buffer offsets): tiles over the range g
    // reaches, with the residue-group size D that minimises a cost model of tap work plus
    // staged elements.
    // D >= min(dil, 4): below that the staging gathers runs of 1-2 complex values with
    // stride dil, a cache line per value (on MI355X such tiles ran up to 2x slower than the
    // model predicts; the weight 48 and this floor come from timing every D on the octaves
    // of the CWT, TokenMixer and attention configurations).
    const int64_t reach = (int64_t)dil * half;
    const int64_t lo = std::min(std::max(x_off - reach, (int64_t)0), n_in);
    const int64_t hi = std::min(std::max(x_off + n_out + reach, lo), n_in);
    const int H = (half + RUN - 1) / RUN * RUN;
    const int64_t nj = std::max((int64_t)1, cdiv(hi - lo, dil));
    int best_d = 0;
    int64_t best_tiles = 0, best_jb = 0;
    double best_cost = 0;
    for (int d = std::min(dil, 4); d <= 64 && d <= dil; d *= 2) {
      const int64_t J = TT / d;
      const int64_t jb = cdiv(nj, J);
      const int64_t tl = (dil / d) * jb;
      const size_t lds = (size_t)(d * (J + 2 * H) * (RUN + 1) / RUN + d) * channels * cs;
      if (lds > 160 * 1024 || tl > INT32_MAX) continue;
      const double cost = (double)tl * ((double)TT * (2 * half + 1) + 48.0 * d * (J + 2 * H)) *
                          channels;
      if (!best_d || cost < best_cost) best_d = d, best_cost = cost, best_tiles = tl, best_jb = jb;
    }
    if (best_d) {
      const int64_t J = TT / best_d;
      const size_t lds =
          (size_t)(best_d * (J + 2 * H) * (RUN + 1) / RUN + best_d) * channels * cs;
#define ADJ(TYPE, CPLX, DD)                                                                  \
  case DD: {                                                                                 \
    auto k = morlet_adjoint_kernel<TYPE, CPLX, DD>;                                          \
    FDWT_LDS_ONCE(k);                                                                        \
    return launch(k, rows * best_tiles, lds, hs, st, (const TYPE*)g, (TYPE*)gx,               \
                  (int)g_scales, (int)best_tiles, (int)best_jb, lo, hi, H, (int)accumulate);  \
  }
#define ADJ_ALL(TYPE, CPLX)                                                                  \
  switch (best_d) {                                                                          \
    ADJ(TYPE, CPLX, 1) ADJ(TYPE, CPLX, 2) ADJ(TYPE, CPLX, 4) ADJ(TYPE, CPLX, 8)              \
    ADJ(TYPE, CPLX, 16) ADJ(TYPE, CPLX, 32) ADJ(TYPE, CPLX, 64) default: break;              \
  }
      if (dtype == FDWT_F32) {
        if (channels == 2) ADJ_ALL(float, true) else ADJ_ALL(float, false)
      } else {
        if (channels == 2) ADJ_ALL(double, true) else ADJ_ALL(double, false)
      }
#undef ADJ_ALL
#undef ADJ
    }
  }
  const int tiles = (int)cdiv(n_in, TT);
  const size_t lds = (size_t)((TT + 2 * (int64_t)dil * half) * channels + 4) * cs;
#define BWX(TYPE, CPLX)                                                                    \
  do {                                                                                      \
    auto k = morlet_backward_x_kernel<TYPE, CPLX>;                                          \
    FDWT_LDS_ONCE(k);                                                                       \
    return launch(k, rows * tiles, lds, hs, st, (const TYPE*)g, (TYPE*)gx, (int)g_scales,    \
                  tiles, (int)accumulate);                                                  \
  } while (0)
  if (dtype == FDWT_F32) {
    if (channels == 2) BWX(float, true);
    BWX(float, false);
  }
  if (channels == 2) BWX(double, true);
  BWX(double, false);
#undef BWX
}

extern "C" int64_t fdwt_morlet_backward_h_workspace(int64_t rows, int64_t n_out, int32_t n_scales,
                                                    int32_t half, int32_t channels) {
  const int64_t tiles = cdiv(n_out, TT);
  return rows * tiles * (int64_t)n_scales * (2 * (int64_t)half + 1) * channels;
}

// The filter gradient with a workspace of workspace_elems elements.  The columns written are
// those of the path taken (resident workgroups on the matrix cores, rows x tiles on the
// vector kernel, each for its own scales when a stage is split between them); a workspace
// smaller than that returns FDWT_ERR_SCRATCH before any launch.
static int morlet_backward_h_run(const void* x, const void* g, void* workspace,
                                 int64_t workspace_elems, void* gh, int64_t rows, int64_t n_in,
                                 int64_t n_out, int64_t x_off, int32_t n_scales, int32_t half,
                                 const int32_t* support, const int32_t* chan, int32_t dil,
                                 int32_t channels, int32_t g_scales, int32_t accumulate,
                                 int32_t dtype, void* stream) {
  Stage st;
  int e = fill_stage(st, x, g, n_in, n_out, x_off, n_scales, half, support, chan, dil, channels);
  if (e) return e;
  // bf16 operands on the matrix-core path; the vector kernel computes in fp32
  const bool bf = dtype == FDWT_F32_BF16;
  if (bf) dtype = FDWT_F32;
  if (!workspace || !gh || rows < 0 || (dtype != FDWT_F32 && dtype != FDWT_F64)) return FDWT_ERR_ARG;
  for (int s = 0; s < n_scales; ++s)
    if (chan[s] >= g_scales) return FDWT_ERR_ARG;
  const int64_t K = 2 * (int64_t)half + 1;
  const int64_t n_el = n_scales * K * channels;
  if (rows == 0 || n_out == 0) return 0;
  if (n_in < 1) return FDWT_ERR_ARG;  // x is staged: a row needs a sample
  const int tiles = (int)cdiv(n_out, TT);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const int cs = dtype == FDWT_F64 ? 8 : 4;
  const int64_t span = TT + 2 * (int64_t)dil * half;
  const int64_t blocks = rows * tiles;
  const size_t vlds = (size_t)(HPAD + ((span + 4 + 3) & ~3) + (int64_t)HS4 * TT * channels) * cs;
  const bool vec_ok = (dil == 1 || dil == 2 || dil % 4 == 0) && n_el <= INT32_MAX;
  int rc = 0;
  // vector kernel over scales [B, E): groups of 4, the remaining 1 or 2 in one smaller group
  // (3 stay in a group of 4, one slot idle); partial rows of scales vfirst.. at stride blocks
  // from element vbase
  int64_t vbase = 0;
  int vfirst = 0;
#define BWH_HS(TYPE, CPLX, D, S, B, E)                                                        \
  do {                                                                                        \
    auto k = morlet_backward_h_kernel<TYPE, CPLX, D, S>;                                      \
    FDWT_LDS_ONCE(k);                                                                         \
    rc = launch(k, blocks, vlds, hs, st, (const TYPE*)g, (TYPE*)workspace + vbase,            \
                (int)g_scales, tiles, (int)(B), (int)(E), vfirst);                            \
  } while (0)
#define BWH_DIL(TYPE, CPLX, D, B, E)                                                          \
  do {                                                                                        \
    const int r4 = ((E) - (B)) % 4, m4 = r4 == 3 ? (E) : (E) - r4;                            \
    if (m4 > (B)) BWH_HS(TYPE, CPLX, D, 4, B, m4);                                            \
    if (!rc && (E) - m4 == 1) BWH_HS(TYPE, CPLX, D, 1, m4, E);                                \
    if (!rc && (E) - m4 == 2) BWH_HS(TYPE, CPLX, D, 2, m4, E);                                \
  } while (0)
#define BWH_RANGE(TYPE, CPLX, B, E)                                                           \
  do {                                                                                        \
    if (dil == 1) BWH_DIL(TYPE, CPLX, 1, B, E);                                               \
    else if (dil == 2) BWH_DIL(TYPE, CPLX, 2, B, E);                                          \
    else BWH_DIL(TYPE, CPLX, 0, B, E);                                                        \
  } while (0)
  // (the matrix-core kernel reads g at 32-bit byte offsets within a row block of g_scales rows)
  const bool a_off_ok = ((int64_t)g_scales * n_out + TT + 64) * channels * cs <= INT32_MAX;
  if (K <= 16 * MB_KB && blocks <= INT32_MAX && a_off_ok) {
    // matrix-core path: launches over groups of 16 / C scales, then one column reduction.  A
    // trailing group of at most GH_VEC_SCALES scales goes to the vector kernel instead: a
    // matrix-core launch costs nearly as much for one scale as for a full group (measured:
    // one scale costs the vector kernel about half a matrix-core launch, two scales as much
    // as or, at dilations 1 and 2 on long rows, 1.4x a matrix-core launch).
    const int kblocks = (int)cdiv(K, 16);
    const int sk = (dil < 8 || (dil & (dil - 1))) ? 30 : __builtin_ctz(dil);
    const int64_t xs = (span + 4 - 1) + 4 * ((span + 4 - 1) >> sk) + 1;
    const size_t mlds = (size_t)std::max<int64_t>(xs, (int64_t)(NT / 64) * kblocks * 256) * cs;
    const int grp = 16 / channels;
    // (the split depends on the shape and operand precision only, never on the workspace
    // size; with bf16 operands a whole group on the matrix cores costs less than one or two
    // scales on the vector kernel, so nothing goes there)
    int tail = n_scales % grp;
    if (tail > GH_VEC_SCALES || !vec_ok || bf) tail = 0;
    const int nm = n_scales - tail;                  // scales on the matrix cores
    const int64_t nm_el = (int64_t)nm * K * channels;  // their filter taps
    int ncols = 0;  // partial columns of the matrix-core rows, then the vector kernel's rows
#define GHM_KB(TYPE, CPLX, N)                                                                 \
  case N: {                                                                                   \
    auto k0 = morlet_grad_h_mfma_kernel<TYPE, CPLX, N, BFV, false>;                           \
    auto k1 = morlet_grad_h_mfma_kernel<TYPE, CPLX, N, BFV, true>;                            \
    FDWT_LDS_ONCE(k0);                                                                        \
    FDWT_LDS_ONCE(k1);                                                                        \
    auto k = sk >= 5 ? k1 : k0;                                                               \
    ncols = resident_blocks(k, mlds, blocks);                                                 \
    if ((int64_t)ncols * nm_el + (n_el - nm_el) * blocks > workspace_elems)                   \
      return FDWT_ERR_SCRATCH;                                                                \
    for (int s0 = 0; s0 < nm && !rc; s0 += grp)                                               \
      rc = launch(k, ncols, mlds, hs, st, (const TYPE*)g, (TYPE*)workspace, (int)g_scales,    \
                  tiles, blocks, s0, std::min(nm, s0 + grp), sk);                             \
    break;                                                                                    \
  }
#define GHM(TYPE, CPLX)                                                                       \
  do {                                                                                        \
    if (nm > 0) {                                                                             \
      switch (kblocks) {                                                                      \
        GHM_KB(TYPE, CPLX, 1) GHM_KB(TYPE, CPLX, 2) GHM_KB(TYPE, CPLX, 3)                     \
        GHM_KB(TYPE, CPLX, 4) GHM_KB(TYPE, CPLX, 5) GHM_KB(TYPE, CPLX, 6)                     \
        GHM_KB(TYPE, CPLX, 7) GHM_KB(TYPE, CPLX, 8) default: return FDWT_ERR_ARG;             \
      }                                                                                       \
    }                                                                                         \
    if (!rc && tail) {                                                                        \
      if (nm == 0 && n_el * blocks > workspace_elems) return FDWT_ERR_SCRATCH;                \
      vbase = nm_el * ncols;                                                                  \
      vfirst = nm;                                                                            \
      BWH_RANGE(TYPE, CPLX, nm, n_scales);                                                    \
    }                                                                                         \
    if (!rc && nm > 0)                                                                        \
      rc = launch(reduce_cols_kernel<TYPE>, nm_el, 0, hs, (const TYPE*)workspace, (TYPE*)gh,  \
                  (int64_t)ncols, (int)accumulate);                                           \
    if (!rc && tail)                                                                          \
      rc = launch(reduce_cols_kernel<TYPE>, n_el - nm_el, 0, hs,                              \
                  (const TYPE*)workspace + vbase, (TYPE*)gh + nm_el, blocks,                  \
                  (int)accumulate);                                                           \
    return rc;                                                                                \
  } while (0)
    if (dtype == FDWT_F32 && bf) {
      constexpr bool BFV = true;
      if (channels == 2) GHM(float, true);
      GHM(float, false);
    }
    constexpr bool BFV = false;
    if (dtype == FDWT_F32) {
      if (channels == 2) GHM(float, true);
      GHM(float, false);
    }
    if (channels == 2) GHM(double, true);
    GHM(double, false);
#undef GHM
#undef GHM_KB
  }
  if (n_el > INT32_MAX) return FDWT_ERR_ARG;
  if (blocks * n_el > workspace_elems) return FDWT_ERR_SCRATCH;
  if (!vec_ok) return FDWT_ERR_ARG;
#define BWH(TYPE, CPLX)                                                                       \
  do {                                                                                        \
    BWH_RANGE(TYPE, CPLX, 0, n_scales);                                                       \
    if (rc) return rc;                                                                        \
    return launch(reduce_cols_kernel<TYPE>, n_el, 0, hs, (const TYPE*)workspace, (TYPE*)gh,   \
                  blocks, (int)accumulate);                                                   \
  } while (0)
  if (dtype == FDWT_F32) {
    if (channels == 2) BWH(float, true);
    BWH(float, false);
  }
  if (channels == 2) BWH(double, true);
  BWH(double, false);
#undef BWH
#undef BWH_RANGE
#undef BWH_DIL
#undef BWH_HS
}

extern "C" int fdwt_morlet_backward_h(const void* x, const void* g, void* workspace,
                                      int64_t workspace_elems, void* gh, int64_t rows,
                                      int64_t n_in, int64_t n_out, int64_t x_off,
                                      int32_t n_scales, int32_t half, const int32_t* support,
                                      const int32_t* chan, int32_t dil, int32_t channels,
                                      int32_t g_scales, int32_t accumulate, int32_t dtype,
                                      void* stream) {
  if (rows < 0 || n_out < 0 || n_scales < 0 || half < 0 || channels < 1) return FDWT_ERR_ARG;
  const int64_t need = fdwt_morlet_backward_h_workspace(rows, n_out, n_scales, half, channels);
  if (workspace_elems < need) return FDWT_ERR_ARG;
  return morlet_backward_h_run(x, g, workspace, workspace_elems, gh, rows, n_in, n_out, x_off,
                               n_scales, half, support, chan, dil, channels, g_scales,
                               accumulate, dtype, stream);
}

// ------------------------------------------------------------------ no-allocation variant
// The filter gradient's partial sums in a fixed device array instead of a caller workspace.
// Host code never passes the array's name to a kernel: its device address is resolved once
// per device (hipGetSymbolAddress, with that device current) and kept in noalloc_ptr.
constexpr int64_t NOALLOC_SCRATCH_BYTES = 32ll << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::once_flag noalloc_once[NOALLOC_MAX_DEVICES];
void* noalloc_ptr[NOALLOC_MAX_DEVICES];
hipError_t noalloc_err[NOALLOC_MAX_DEVICES];

// device address of the current device's copy of `scratch`
int noalloc_scratch(void** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return FDWT_ERR_ARG;
  std::call_once(noalloc_once[dev], [dev] {
    noalloc_err[dev] = hipGetSymbolAddress(&noalloc_ptr[dev], HIP_SYMBOL(scratch));
  });
  if (noalloc_err[dev] != hipSuccess) return (int)noalloc_err[dev];
  if (!noalloc_ptr[dev]) return FDWT_ERR_ARG;
  *out = noalloc_ptr[dev];
  return 0;
}
}  // namespace

extern "C" int64_t fdwt_morlet_backward_h_noalloc_capacity(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int fdwt_morlet_backward_h_noalloc(const void* x, const void* g, void* gh,
                                              int64_t rows, int64_t n_in, int64_t n_out,
                                              int64_t x_off, int32_t n_scales, int32_t half,
                                              const int32_t* support, const int32_t* chan,
                                              int32_t dil, int32_t channels, int32_t g_scales,
                                              int32_t accumulate, int32_t dtype, void* stream) {
  if (dtype != FDWT_F32 && dtype != FDWT_F64 && dtype != FDWT_F32_BF16) return FDWT_ERR_ARG;
  void* ws = nullptr;
  const int e = noalloc_scratch(&ws);
  if (e) return e;
  // every column the kernels read back is written first by the same call: nothing to clear
  const int64_t elems = NOALLOC_SCRATCH_BYTES / (dtype == FDWT_F64 ? 8 : 4);
  return morlet_backward_h_run(x, g, ws, elems, gh, rows, n_in, n_out, x_off, n_scales, half,
                               support, chan, dil, channels, g_scales, accumulate, dtype,
                               stream);
}

extern "C" int64_t fdwt_mix_workspace(int64_t rows, int64_t n_out, int32_t n_scales) {
  return rows * cdiv(n_out, TT) * (int64_t)n_scales * 2;
}

extern "C" int fdwt_mix_forward(const void* x, const void* taps, const void* a, const void* b,
                                void* y, int64_t rows, int64_t n_in, int64_t n_out,
                                int64_t x_off, int32_t n_scales, int32_t half,
                                const int32_t* support, const int32_t* chan, int32_t dil,
                                int32_t channels, int32_t s_total, int32_t d_dim, int64_t row0,
                                int32_t accumulate, int32_t dtype, void* stream) {
  Stage st;
  int e = fill_stage(st, x, taps, n_in, n_out, x_off, n_scales, half, support, chan, dil, channels);
  if (e) return e;
  if (!a || !b || !y || rows < 0 || d_dim < 1 || row0 < 0 || (dtype != FDWT_F32 && dtype != FDWT_F64))
    return FDWT_ERR_ARG;
  for (int s = 0; s < n_scales; ++s)
    if (chan[s] >= s_total) return FDWT_ERR_ARG;
  if (rows == 0 || n_out == 0) return 0;
  if (n_in < 1) return FDWT_ERR_ARG;  // x is staged: a row needs a sample
  const int tiles = (int)cdiv(n_out, TT);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const int cs = dtype == FDWT_F64 ? 8 : 4;
  const size_t lds = tile_lds(st, cs, 16);
#define MIXF(TYPE, CPLX)                                                                      \
  do {                                                                                        \
    auto k = mix_kernel<TYPE, CPLX, false>;                                                   \
    FDWT_LDS_ONCE(k);                                                                         \
    return launch(k, rows * tiles, lds, hs, st, (const TYPE*)a, (const TYPE*)b, (int)s_total,  \
                  (int)d_dim, row0, (TYPE*)y, (const TYPE*)nullptr, (TYPE*)nullptr,           \
                  (TYPE*)nullptr, tiles, (int)accumulate);                                    \
  } while (0)
  if (dtype == FDWT_F32) {
    if (channels == 2) MIXF(float, true);
    MIXF(float, false);
  }
  if (channels == 2) MIXF(double, true);
  MIXF(double, false);
#undef MIXF
}

extern "C" int fdwt_mix_backward(const void* x, const void* taps, const void* a, const void* b,
                                 const void* gy, void* gw, void* workspace,
                                 int64_t workspace_elems, int64_t rows, int64_t n_in,
                                 int64_t n_out, int64_t x_off, int32_t n_scales, int32_t half,
                                 const int32_t* support, const int32_t* chan, int32_t dil,
                                 int32_t channels, int32_t s_total, int32_t d_dim, int64_t row0,
                                 int32_t dtype, void* stream) {
  Stage st;
  int e = fill_stage(st, x, taps, n_in, n_out, x_off, n_scales, half, support, chan, dil, channels);
  if (e) return e;
  if (!a || !b || !gy || !gw || !workspace || rows < 0 || d_dim < 1 || row0 < 0 ||
      (dtype != FDWT_F32 && dtype != FDWT_F64))
    return FDWT_ERR_ARG;
  for (int s = 0; s < n_scales; ++s)
    if (chan[s] >= s_total) return FDWT_ERR_ARG;
  if (workspace_elems < fdwt_mix_workspace(rows, n_out, n_scales)) return FDWT_ERR_ARG;
  if (rows == 0 || n_out == 0) return 0;
  if (n_in < 1) return FDWT_ERR_ARG;  // x is staged: a row needs a sample
  const int tiles = (int)cdiv(n_out, TT);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const int cs = dtype == FDWT_F64 ? 8 : 4;
  const size_t lds = tile_lds(st, cs, 16);
  // the workspace receives per-(row, tile) partial sums (rows, tiles, n_scales, 2); the
  // caller reduces the rows that share a weight row d in a fixed order
#define MIXB(TYPE, CPLX)                                                                      \
  do {                                                                                        \
    auto k = mix_kernel<TYPE, CPLX, true>;                                                    \
    FDWT_LDS_ONCE(k);                                                                         \
    return launch(k, rows * tiles, lds, hs, st, (const TYPE*)a, (const TYPE*)b, (int)s_total,  \
                  (int)d_dim, row0, (TYPE*)nullptr, (const TYPE*)gy, (TYPE*)gw,               \
                  (TYPE*)workspace, tiles, 0);                                                \
  } while (0)
  if (dtype == FDWT_F32) {
    if (channels == 2) MIXB(float, true);
    MIXB(float, false);
  }
  if (channels == 2) MIXB(double, true);
  MIXB(double, false);
#undef MIXB
}

extern "C" int fdwt_softmax_forward(const void* x, const void* taps, const void* v,
                                    int32_t v_per_position, int64_t v_s_total, int32_t nch,
                                    void* m, void* l, void* num, int64_t rows, int64_t n_in,
                                    int64_t n_out, int64_t x_off, int32_t n_scales, int32_t half,
                                    const int32_t* support, const int32_t* chan, int32_t dil,
                                    double inv_tau, int32_t first, int32_t last, int32_t dtype,
                                    void* stream) {
  Stage st;
  int e = fill_stage(st, x, taps, n_in, n_out, x_off, n_scales, half, support, chan, dil, 2);
  if (e) return e;
  if (!v || !m || !l || !num || rows < 0 || nch < 1 || (dtype != FDWT_F32 && dtype != FDWT_F64))
    return FDWT_ERR_ARG;
  for (int s = 0; s < n_scales; ++s)
    if (chan[s] >= v_s_total) return FDWT_ERR_ARG;
  if (rows == 0 || n_out == 0) return 0;
  if (n_in < 1) return FDWT_ERR_ARG;  // x is staged: a row needs a sample
  SoftArgs sa{v, v_s_total, nch, v_per_position ? 1 : 0, 0, inv_tau};
  const int tiles = (int)cdiv(n_out, TT);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const int cs = dtype == FDWT_F64 ? 8 : 4;
  const size_t lds = tile_lds(st, cs, 0);
  if (dtype == FDWT_F32) {
    auto k = softmax_forward_kernel<float>;
    FDWT_LDS_ONCE(k);
    return launch(k, rows * tiles, lds, hs, st, sa, (float*)m, (float*)l, (float*)num, tiles,
                  (int)first, (int)last);
  }
  auto k = softmax_forward_kernel<double>;
  FDWT_LDS_ONCE(k);
  return launch(k, rows * tiles, lds, hs, st, sa, (double*)m, (double*)l, (double*)num, tiles,
                (int)first, (int)last);
}

extern "C" int64_t fdwt_softmax_workspace(int64_t rows, int64_t n_out, int32_t n_scales,
                                          int32_t v_per_position) {
  if (v_per_position) return rows * (int64_t)n_scales * n_out;
  return rows * cdiv(n_out, TT) * (int64_t)n_scales;
}

extern "C" int fdwt_softmax_dv_reduce(const void* part, void* gv, int64_t groups, int32_t nch,
                                      int32_t n_scales, const int32_t* chan, int64_t v_groups,
                                      int64_t v_s_total, int64_t n_out, int64_t g0,
                                      int32_t dtype, void* stream) {
  if (!part || !gv || !chan || groups < 0 || nch < 1 || n_scales < 0 || n_scales > MAXS ||
      v_s_total < 1 || n_out < 0 || g0 < 0 || g0 + groups > v_groups ||
      (dtype != FDWT_F32 && dtype != FDWT_F64))
    return FDWT_ERR_ARG;
  DvArgs ca{};
  for (int s = 0; s < n_scales; ++s) {
    if (chan[s] < 0 || chan[s] >= v_s_total) return FDWT_ERR_ARG;
    ca.chan[s] = chan[s];
  }
  if (groups == 0 || n_scales == 0 || n_out == 0) return 0;
  const int64_t tiles = cdiv(n_out, NT);
  const int64_t blocks = groups * n_scales * tiles;
  if (tiles > INT32_MAX || blocks > INT32_MAX) return FDWT_ERR_ARG;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (dtype == FDWT_F32)
    return launch(softmax_dv_kernel<float>, blocks, 0, hs, (const float*)part, (float*)gv, ca,
                  (int)nch, (int)n_scales, v_s_total, n_out, g0, (int)tiles);
  return launch(softmax_dv_kernel<double>, blocks, 0, hs, (const double*)part, (double*)gv, ca,
                (int)nch, (int)n_scales, v_s_total, n_out, g0, (int)tiles);
}

extern "C" int fdwt_softmax_backward(const void* x, const void* taps, const void* v,
                                     int32_t v_per_position, int64_t v_s_total, int32_t nch,
                                     int64_t row0, const void* m, const void* l, const void* out,
                                     const void* gy, void* gw, void* workspace,
                                     int64_t workspace_elems, int64_t rows, int64_t n_in,
                                     int64_t n_out, int64_t x_off, int32_t n_scales, int32_t half,
                                     const int32_t* support, const int32_t* chan, int32_t dil,
                                     double inv_tau, int32_t dtype, void* stream) {
  Stage st;
  int e = fill_stage(st, x, taps, n_in, n_out, x_off, n_scales, half, support, chan, dil, 2);
  if (e) return e;
  if (!v || !m || !l || !out || !gy || !gw || !workspace || rows < 0 || nch < 1 || row0 < 0 ||
      (dtype != FDWT_F32 && dtype != FDWT_F64))
    return FDWT_ERR_ARG;
  for (int s = 0; s < n_scales; ++s)
    if (chan[s] >= v_s_total) return FDWT_ERR_ARG;
  if (workspace_elems < fdwt_softmax_workspace(rows, n_out, n_scales, v_per_position))
    return FDWT_ERR_ARG;
  if (rows == 0 || n_out == 0) return 0;
  if (n_in < 1) return FDWT_ERR_ARG;  // x is staged: a row needs a sample
  SoftArgs sa{v, v_s_total, nch, v_per_position ? 1 : 0, row0, inv_tau};
  const int tiles = (int)cdiv(n_out, TT);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const int cs = dtype == FDWT_F64 ? 8 : 4;
  const size_t lds = tile_lds(st, cs, 16);
  if (dtype == FDWT_F32) {
    auto k = softmax_backward_kernel<float>;
    FDWT_LDS_ONCE(k);
    return launch(k, rows * tiles, lds, hs, st, sa, (const float*)m, (const float*)l,
                  (const float*)out, (const float*)gy, (float*)gw, (float*)workspace, tiles);
  }
  auto k = softmax_backward_kernel<double>;
  FDWT_LDS_ONCE(k);
  return launch(k, rows * tiles, lds, hs, st, sa, (const double*)m, (const double*)l,
                (const double*)out, (const double*)gy, (double*)gw, (double*)workspace, tiles);
}


// ------------------------------------------------------------------ filter synthesis (host)
static int fill_filter_args(FilterArgs& fa, const double* scales, const double* w0,
                            const int32_t* dil, const int32_t* support, int32_t n_scales,
                            int32_t center, int32_t channels, int32_t norm_l2, int32_t dtype) {
  if (!scales || !w0 || !dil || !support || n_scales < 1 || n_scales > MAXF || center < 0 ||
      (channels != 1 && channels != 2) || (dtype != FDWT_F32 && dtype != FDWT_F64))
    return FDWT_ERR_ARG;
  fa.scales = scales;
  fa.w0 = w0;
  fa.n_scales = n_scales;
  fa.center = center;
  fa.C = channels;
  fa.l2 = norm_l2 ? 1 : 0;
  for (int i = 0; i < MAXF; ++i) {
    fa.dil[i] = i < n_scales ? dil[i] : 1;
    fa.sup[i] = i < n_scales ? support[i] : 0;
    if (i < n_scales && (dil[i] < 1 || support[i] < 0)) return FDWT_ERR_ARG;
  }
  return 0;
}

extern "C" int fdwt_morlet_filters(const double* scales, const double* w0, const int32_t* dil,
                                   const int32_t* support, int32_t n_scales, int32_t center,
                                   int32_t channels, int32_t norm_l2, void* H, int32_t dtype,
                                   void* stream) {
  FilterArgs fa;
  int e = fill_filter_args(fa, scales, w0, dil, support, n_scales, center, channels, norm_l2,
                           dtype);
  if (e) return e;
  if (!H) return FDWT_ERR_ARG;
  const int64_t blocks = cdiv((int64_t)n_scales * (center + 1), NT);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (dtype == FDWT_F32) return launch(morlet_filters_kernel<float>, blocks, 0, hs, fa, (float*)H);
  return launch(morlet_filters_kernel<double>, blocks, 0, hs, fa, (double*)H);
}

extern "C" int fdwt_morlet_filters_backward(const double* scales, const double* w0,
                                            const int32_t* dil, const int32_t* support,
                                            int32_t n_scales, int32_t center, int32_t channels,
                                            int32_t norm_l2, const void* gH, int32_t dtype,
                                            double* g_scales, double* g_w0, void* stream) {
  FilterArgs fa;
  int e = fill_filter_args(fa, scales, w0, dil, support, n_scales, center, channels, norm_l2,
                           dtype);
  if (e) return e;
  if (!gH || !g_scales || !g_w0) return FDWT_ERR_ARG;
  hipStream_t hs = static_cast<hipStream_t>(stream);
  if (dtype == FDWT_F32)
    return launch(morlet_filters_backward_kernel<float>, 1, 0, hs, fa, (const float*)gH,
                  g_scales, g_w0);
  return launch(morlet_filters_backward_kernel<double>, 1, 0, hs, fa, (const double*)gH,
                g_scales, g_w0);
}

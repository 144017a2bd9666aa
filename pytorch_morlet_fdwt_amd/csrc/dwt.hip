// Mallat DWT kernels for gfx950: analysis (two bands, stride-2) and its exact transpose.
//
// Analysis of one level (reference semantics: src/fdwt/kernels/dwt.py:73-98):
//     y_b[o] = sum_{j<L} h_b[j] x_ext[2 o + off - j]
// Synthesis is the transpose: z[p] = sum_{2o + off - j = p} h0[j] a[o] + h1[j] d[o] for the
// extended positions p, then every z[p] is folded back onto y[ext(p)] (dwt.py:101-175).
//
// Design (MI355X-first, not a translation of the Triton kernels):
//  * Boundary extension is applied only when a signal is staged into LDS (or when its
//    margins are filled); the tap loops read a branch-free, already extended window.
//  * Each thread computes V consecutive outputs from a register window (2V + L - 2 samples
//    for analysis, V + L/2 - 1 coefficients per band for synthesis); taps live in SGPRs.
//  * Fused chains: one workgroup owns one row, and the low band of every level stays in LDS
//    (ping-pong buffers), so the input is read once and each band is written once.
//    Level 0 of an analysis chain streams x through an LDS window whose next chunk is
//    prefetched into registers while the current chunk is computed.
//  * Split kernels (one level, several workgroups per row) serve rows too long for LDS.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.h"

namespace fdwt {
namespace {

constexpr int NT = 512;          // threads per workgroup (8 wave64): two resident rows per
                                 // CU then keep enough loads in flight to cover HBM latency
constexpr int VA = 2;            // consecutive analysis outputs per thread
constexpr int GA = 2;            // thread groups per analysis chunk
constexpr int CO = NT * VA * GA; // outputs per analysis chunk (2048)
constexpr int VS = 2;            // consecutive synthesis pairs (u values) per thread
constexpr int GS = 5;            // thread groups per synthesis pass
constexpr int PS = NT * VS * GS; // coefficient pairs per synthesis pass (split kernel)
constexpr int VR = 4;            // consecutive synthesis pairs per thread (whole-row kernel)
constexpr int GR = 3;            // thread groups per pass (whole-row kernel)
constexpr int PR = NT * VR * GR; // coefficient pairs per pass of the whole-row kernel (6144)
constexpr int QR = 16;           // queue registers per thread (queue <= QR * NT samples)
constexpr int MAXL_T = 32;       // largest templated filter length
constexpr int MAX_TAPS = 256;    // longest filter accepted (PyWavelets' longest is 102)

struct AChainArgs {
  const void* x;
  void* details[FDWT_MAX_LEVELS];
  void* approx;
  const void* h0;
  const void* h1;
  int32_t n_in[FDWT_MAX_LEVELS];
  int32_t n_out[FDWT_MAX_LEVELS];
  int32_t levels, taps, mode, off;
  int32_t capA, capB;
  int32_t split;  // chunks per workgroup in split mode (levels == 1), 0 = whole row
};

struct SChainArgs {
  const void* approx;
  const void* details[FDWT_MAX_LEVELS];
  void* out;
  const void* h0;
  const void* h1;
  int32_t nc[FDWT_MAX_LEVELS];
  int32_t n_out[FDWT_MAX_LEVELS];
  int32_t levels, taps, mode, off;
  int32_t capA, capB, capE, capD;
  int32_t split;  // output positions per workgroup in split mode (levels == 1), 0 = row
  // whole-row workgroups: first coefficient pair of each level's passes
  int32_t ub0[FDWT_MAX_LEVELS];
  // the "queue": the high bands of the first qlevels levels (each a single pass), loaded into
  // QR register slots of NT coefficients at kernel start.  Slot k holds coefficients
  // qs_u0[k] .. qs_u0[k] + NT - 1 of the band qs_ptr[k] (rows of qs_nc[k] coefficients);
  // level l < qlevels uses slots qs0[l] .. qs0[l] + qsn[l] - 1, of which its pass reads the
  // first qlen[l] coefficients
  const void* qs_ptr[QR];
  int32_t qs_nc[QR];
  int32_t qs_u0[QR];
  int32_t qs0[FDWT_MAX_LEVELS];
  int32_t qsn[FDWT_MAX_LEVELS];
  int32_t qlen[FDWT_MAX_LEVELS];
  int32_t qslots;
  int32_t qlevels;
};

// ------------------------------------------------------------------ persistent synthesis: plan
// The whole-row synthesis kernel (one workgroup per row at a time, rows blockIdx.x,
// blockIdx.x + gridDim.x, ...) keeps the low band of every level in LDS and reads each band of
// a row from HBM exactly once, into prefetch registers, well before it is used.  A prefetch
// register holds up to PQ NT consecutive coefficients of one band (lane t the coefficients
// t + j NT, j < PQ: every load and LDS store of the register is coalesced), loaded through a
// buffer resource whose range is the register's coefficients (lanes past the end read 0), so a
// register costs one descriptor read and no per-lane address arithmetic.  Two register sets:
//  * the head (PA registers): every band of the levels before the last (a_0, d_0 .. d_{J-2}),
//    requested for the next row just before the current row's last level runs;
//  * the tail (PB registers): the last level's band(s), requested at the start of the row, so
//    that it arrives while levels 0 .. J-2 run.
// The kernel waits for outstanding loads explicitly at two points only (the start of a row and
// the start of its last level); in between, staging reads registers whose loads are known to
// be complete, so the compiler adds no wait of its own.  Rows whose bands do not fit the sets
// load each band at its level instead (no prefetch).
constexpr int PQ = 4;  // coefficients per lane in one prefetch register
constexpr int PA = 9;  // head prefetch registers per thread (2- and 4-byte bands)
constexpr int PB = 5;  // tail prefetch registers per thread
// head registers for bands of es-byte coefficients (8-byte ones take twice the VGPRs)
__host__ __device__ constexpr int syn_pa(int es) { return es == 8 ? 6 : PA; }

// LDS buffers of the whole-row synthesis kernel, in this order (element offsets P, Q, D, E,
// T): the low band of level l lives in P when J - 1 - l is even and in Q otherwise (the last
// level reads P); the high band of levels < J - 1 is staged in D and the last level's high
// band across Q and D, which hold nothing live by then.  E holds the positions parked for the
// boundary fold, T the taps of runtime-length filters.
inline int syn_src(int l, int J, int P, int Q) { return ((J - 1 - l) & 1) ? Q : P; }
inline int syn_dbuf(int l, int J, int Q, int D) { return l == J - 1 ? Q : D; }

// Geometry of one synthesis level.  The level produces z(p) for the extended positions
// p in [pbeg, pend) from the coefficient pairs v in [vbeg, vend) (pair v gives positions
// 2v + off - 1 and 2v + off).  Positions in [plo, phi) are written as they are; the others are
// parked in E and, after the level, every fold target i in [0, plo) or [phi, mw) receives the
// sum of the parked values of the positions that the mode's extension maps onto it.  Zero
// mode folds nothing (plo = 0, phi = mw).  mw = positions the next level reads (all m on the
// last level).  The level reads coefficients [vbeg - .., zhi) of both bands (zero outside the
// band).
struct SynGeom {
  int m, mw, md, P, pbeg, pend, plo, phi, vbeg, vend, zhi, ne, nt;
};

__host__ __device__ inline int floor_div(int a, int b) {
  return a >= 0 ? a / b : -((-a + b - 1) / b);
}

__host__ __device__ inline SynGeom syn_geom(int nc, int m, int ncn, bool last, int L, int off,
                                            int mode) {
  SynGeom g;
  g.m = m;
  g.md = normalize_mode(mode, m);
  g.P = mode_period(g.md, m);
  g.mw = last ? m : (ncn < m ? ncn : m);
  const int pmin = off - (L - 1);
  const int pmax = 2 * (nc - 1) + off;
  if (g.md == FDWT_MODE_ZERO) {
    g.pbeg = 0;
    g.pend = g.mw;
    g.plo = 0;
    g.phi = g.mw;
  } else {
    const int nleft = pmin < 0 ? -pmin : 0;
    const int nright = pmax - m + 1 > 0 ? pmax - m + 1 : 0;
    // every extended position folds onto a position within max(nleft, nright) + 1 of an end
    const int band = (nleft > nright ? nleft : nright) + 2;
    g.pbeg = pmin < 0 ? pmin : 0;
    g.pend = pmax + 1 > m ? pmax + 1 : m;
    if (m <= 2 * band) {
      g.plo = m;
      g.phi = m;
    } else {
      g.plo = band;
      g.phi = m - band < g.mw ? m - band : g.mw;
      if (g.phi < g.plo) g.phi = g.plo;
    }
  }
  g.ne = (g.plo - g.pbeg) + (g.pend - g.phi);
  const int nl = g.plo < g.mw ? g.plo : g.mw;
  g.nt = nl + (g.mw > g.phi ? g.mw - g.phi : 0);
  g.vbeg = floor_div(floor_div(g.pbeg - off + 1, 2), VR) * VR;
  g.vend = floor_div(g.pend - off, 2) + 1;
  if (g.vend < g.vbeg) g.vend = g.vbeg;
  g.zhi = (((g.vend > nc ? g.vend : nc) + VR + L / 2 + 4) + 3) & ~3;
  return g;
}

// Per-level record of the kernel (80 bytes).
struct SynLevel {
  int32_t m, mw, md, P;
  int32_t pbeg, pend, plo, phi;
  int32_t vbeg, vend, zhi, nt;
  int32_t src, dst, dbuf, nva;  // buffer offsets (dst -1 on the last level); valid low-band
  int32_t nvd, pad[3];          // coefficients; valid high-band coefficients
};

// One prefetch register: up to NT consecutive coefficients of one band, lane t holding the
// t-th; its load descriptor (16 bytes) and staging word.
struct SynLoad {
  const void* base;  // lane 0's coefficient in row 0
  int32_t stride;    // bytes per row of the band
  int32_t cnt;       // coefficients held (0: register unused)
};
// Staging word of a prefetch register: LDS element offset of lane 0's coefficient | count << 18.
__host__ __device__ inline uint32_t syn_stage_word(int dest, int cnt) {
  return (uint32_t)dest | ((uint32_t)cnt << 18);
}

// Tables of the whole-row synthesis kernel, passed in the kernel arguments and copied to LDS
// by each workgroup once: the kernel reads them at every level and row, and LDS reads (a
// broadcast address) are far cheaper than scalar loads of the argument segment.
struct SynTab {
  uint32_t maskA[FDWT_SYN_MAX_LEVELS];  // head registers staged at each level
  SynLevel lv[FDWT_SYN_MAX_LEVELS];
  SynLoad ldA[PA];  // head registers
  SynLoad ldB[PB];  // tail registers
  uint32_t stA[PA];
  uint32_t stB[PB];
  uint32_t stpad[2];
};
static_assert(sizeof(SynTab) % 16 == 0, "the LDS copy uses whole 16-byte words");

// Arguments of the whole-row synthesis kernel.
struct SynArgs {
  // band[0] = the coarsest approximation, band[l + 1] = the details of level l (one array: a
  // run-time choice between two argument fields would make the compiler copy the arguments to
  // private memory)
  const void* band[FDWT_SYN_MAX_LEVELS + 1];
  void* out;
  const void* h0;
  const void* h1;
  int64_t rows;
  int32_t nc[FDWT_SYN_MAX_LEVELS];
  int32_t levels, taps, off, prefetch;  // prefetch: the bands fit the head and tail registers
  int32_t offE, offTap;
  SynTab tab;
};

// The prefetch registers of a row: each band of the head (a_0, d_0 .. d_{J-2} when J > 1)
// and of the tail (d_{J-1}, or a_0 and d_0 when J == 1) takes ceil(count / per) registers of
// its set (per = PQ NT coefficients; pa, pb registers in the sets).  emit(tail, k, c0, cnt,
// dest, level, is_approx) is called for each register; returns false when a set overflows
// (then nothing is prefetched).
template <typename F>
inline bool syn_regs(int J, const int32_t* nc, const void* approx, const void* const* details,
                     int ZL, int yP, int yQ, int yD, int per, int pa, int pb, F&& emit) {
  int ka = 0, kb = 0;
  for (int s = 0; s <= J; ++s) {
    const int l = s == 0 ? 0 : s - 1;
    const void* ptr = s == 0 ? approx : details[l];
    const int cnt = nc[l];
    if (!ptr || cnt <= 0) continue;
    const bool tail = l == J - 1;
    const int dest = (s == 0 ? syn_src(0, J, yP, yQ) : syn_dbuf(l, J, yQ, yD)) + ZL;
    for (int c0 = 0; c0 < cnt; c0 += per) {
      int& k = tail ? kb : ka;
      if (k == (tail ? pb : pa)) return false;
      emit(tail, k, c0, cnt - c0 < per ? cnt - c0 : per, dest + c0, l, s == 0);
      ++k;
    }
  }
  return true;
}

// Load element i of a global array whose pointer the compiler cannot place in the global
// address space (e.g. one read from LDS): a generic (flat) load would also count against the
// LDS wait counter, so every later LDS wait would wait for it too.
// One 16-byte-aligned group of four floats through a global (not flat) pointer.
typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
__device__ inline v4u_t global_load16(const float* p) {
  typedef __attribute__((address_space(1))) const v4u_t* gptr;
  return *(gptr)p;
}

// One coefficient through a buffer resource (0 outside its range), as raw storage bits.
template <typename S>
__device__ inline S buffer_load_raw(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  S v;
  if constexpr (sizeof(S) == 2) {
    const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
    __builtin_memcpy(&v, &u, 2);
  } else if constexpr (sizeof(S) == 4) {
    const unsigned u = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    __builtin_memcpy(&v, &u, 4);
  } else {
    const auto u = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    __builtin_memcpy(&v, &u, 8);
  }
  return v;
}

template <typename S>
__device__ inline S global_load(const S* p, int64_t i) {
  typedef typename std::conditional<
      sizeof(S) == 2, uint16_t,
      typename std::conditional<sizeof(S) == 4, uint32_t, uint64_t>::type>::type U;
  typedef __attribute__((address_space(1))) const U* gptr;
  const U u = ((gptr)p)[i];
  S v;
  __builtin_memcpy(&v, &u, sizeof(S));
  return v;
}

// Read a record that every lane reads at the same LDS address and make it wave-uniform.
template <typename R>
__device__ inline R lds_uniform(const R* p) {
  static_assert(sizeof(R) % 16 == 0, "records are whole 16-byte words");
  typedef int v4i __attribute__((ext_vector_type(4)));
  const v4i* q = reinterpret_cast<const v4i*>(p);
  int w[sizeof(R) / 4];
#pragma unroll
  for (int k = 0; k < (int)sizeof(R) / 16; ++k) {
    const v4i t = q[k];
    w[4 * k + 0] = __builtin_amdgcn_readfirstlane(t.x);
    w[4 * k + 1] = __builtin_amdgcn_readfirstlane(t.y);
    w[4 * k + 2] = __builtin_amdgcn_readfirstlane(t.z);
    w[4 * k + 3] = __builtin_amdgcn_readfirstlane(t.w);
  }
  R r;
  __builtin_memcpy(&r, w, sizeof(R));
  return r;
}

// Per-level parameters of the synthesis chain as the kernel keeps them in LDS (64 bytes).
struct LevelRec {
  int32_t nc, n_out, ub0, qs0, qsn, qlen, ncn, pad;
  const void* drow;  // this workgroup's row of the level's high band, or null
  int32_t pad2[6];
};
constexpr int LREC_BYTES = FDWT_MAX_LEVELS * (int)sizeof(LevelRec);

// Read one LevelRec (same address in every lane) and make its fields wave-uniform.
__device__ inline LevelRec load_level(const LevelRec* p) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  const v4i a = reinterpret_cast<const v4i*>(p)[0];
  const v4i b = reinterpret_cast<const v4i*>(p)[1];
  const v4i c = reinterpret_cast<const v4i*>(p)[2];
  LevelRec r;
  r.nc = __builtin_amdgcn_readfirstlane(a.x);
  r.n_out = __builtin_amdgcn_readfirstlane(a.y);
  r.ub0 = __builtin_amdgcn_readfirstlane(a.z);
  r.qs0 = __builtin_amdgcn_readfirstlane(a.w);
  r.qsn = __builtin_amdgcn_readfirstlane(b.x);
  r.qlen = __builtin_amdgcn_readfirstlane(b.y);
  r.ncn = __builtin_amdgcn_readfirstlane(b.z);
  r.pad = 0;
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane(c.x);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane(c.y);
  r.drow = reinterpret_cast<const void*>(lo | (hi << 32));
  return r;
}

// ------------------------------------------------------------------ compute windows
// Read W consecutive LDS elements starting at an address aligned to V elements with V-wide
// vector loads (ds_read_b64 / ds_read_b128); neighbouring lanes then read neighbouring
// words, which keeps the access free of bank conflicts.  May read up to V - 1 elements past
// the window.
template <int V, typename T, int W>
__device__ inline void lds_window(const T* __restrict__ p, T (&w)[W]) {
  typedef T vec __attribute__((ext_vector_type(V)));
  const vec* q = reinterpret_cast<const vec*>(p);
#pragma unroll
  for (int v = 0; v < (W + V - 1) / V; ++v) {
    const vec t = q[v];
#pragma unroll
    for (int e = 0; e < V; ++e)
      if (V * v + e < W) w[V * v + e] = t[e];
  }
}

// VA consecutive analysis outputs of both bands from the extended window s (16-byte
// aligned): y_b[q] = sum_i hr_b[i] s[2 q + i] with hr_b the reversed filter.
template <typename T, int LT>
__device__ inline void analysis_pair(const T* __restrict__ s, const T* hr0, const T* hr1,
                                     int L, T (&y0)[VA], T (&y1)[VA]) {
  if constexpr (LT > 0) {
    constexpr int W = 2 * VA + LT - 2;
    T w[W];
    lds_window<(sizeof(T) == 4 ? 4 : 2)>(s, w);  // windows start 2 * VA = 4 elements apart
#pragma unroll
    for (int q = 0; q < VA; ++q) {
      T a0 = T(0), a1 = T(0);
#pragma unroll
      for (int i = 0; i < LT; ++i) {
        a0 = fma(hr0[i], w[2 * q + i], a0);
        a1 = fma(hr1[i], w[2 * q + i], a1);
      }
      y0[q] = a0;
      y1[q] = a1;
    }
  } else {
#pragma unroll
    for (int q = 0; q < VA; ++q) {
      T a0 = T(0), a1 = T(0);
      for (int i = 0; i < L; ++i) {
        const T v = s[2 * q + i];
        a0 = fma(hr0[i], v, a0);
        a1 = fma(hr1[i], v, a1);
      }
      y0[q] = a0;
      y1[q] = a1;
    }
  }
}

// z_odd[q] (position off + 2(u0+q) - 1) and z_even[q] (position off + 2(u0+q)) from the
// low band a[0..] and the high band d[0..], both LDS windows starting at coefficient u0
// (16-byte aligned, zero outside the coefficients).
template <typename T, int LT, int V = VS>
__device__ inline void synthesis_block(const T* __restrict__ a, const T* __restrict__ d,
                                       const T* h0, const T* h1, int L, T (&zo)[V],
                                       T (&ze)[V]) {
  if constexpr (LT > 0) {
    constexpr int H = LT / 2;
    constexpr int W = V + H - 1;
    T av[W], dv[W];
    // windows start V elements apart: vector reads of 4 or 2, single words for odd V
    constexpr int WV = (V >= 4 && sizeof(T) == 4) ? 4 : (V % 2 == 0 ? 2 : 1);
    lds_window<WV>(a, av);
    lds_window<WV>(d, dv);
#pragma unroll
    for (int q = 0; q < V; ++q) {
      T so = T(0), se = T(0);
#pragma unroll
      for (int t = 0; t < H; ++t) {
        se = fma(h0[2 * t], av[q + t], se);
        se = fma(h1[2 * t], dv[q + t], se);
        so = fma(h0[2 * t + 1], av[q + t], so);
        so = fma(h1[2 * t + 1], dv[q + t], so);
      }
      zo[q] = so;
      ze[q] = se;
    }
  } else {
    const int H = L / 2;
#pragma unroll
    for (int q = 0; q < V; ++q) {
      T so = T(0), se = T(0);
      for (int t = 0; t < H; ++t) {
        const T av = a[q + t];
        const T dv = d[q + t];
        se = fma(h0[2 * t], av, se);
        se = fma(h1[2 * t], dv, se);
        so = fma(h0[2 * t + 1], av, so);
        so = fma(h1[2 * t + 1], dv, so);
      }
      zo[q] = so;
      ze[q] = se;
    }
  }
}

// Value of z at one extended position p (used for the few positions outside [0, n) that are
// folded back).  The low band comes from LDS (a_lds[u], zero margins) or, when a_lds is
// null, from the global row a_glob (null = zeros); d from the global row drow (null = zeros).
template <typename S, typename T>
__device__ inline T synthesis_point(const T* __restrict__ a_lds, const S* __restrict__ a_glob,
                                    const S* __restrict__ drow, int p, int off, int nc,
                                    const T* h0, const T* h1, int L) {
  const int r = p - off;
  const int par = r & 1;            // odd r: taps 2t + 1
  const int u = (r + par) >> 1;     // floor division for negative r as well
  T z = T(0);
  // taps in batches of 8 whose (clamped, unconditional) global loads are all in flight
  // together; out-of-range coefficients are zeroed by select
  for (int t0 = 0; t0 < L / 2; t0 += 8) {
    T av[8], dv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int o = u + t0 + k;
      const int oc = min(max(o, 0), nc - 1);
      const bool ok = o >= 0 && o < nc && t0 + k < L / 2;
      T a = a_lds ? a_lds[oc] : (a_glob ? T(Storage<S>::load(a_glob, oc)) : T(0));
      T d = drow ? T(Storage<S>::load(drow, oc)) : T(0);
      av[k] = ok ? a : T(0);
      dv[k] = ok ? d : T(0);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (t0 + k < L / 2) {
        z = fma(h0[2 * (t0 + k) + par], av[k], z);
        z = fma(h1[2 * (t0 + k) + par], dv[k], z);
      }
    }
  }
  return z;
}

// init + sum of the out-of-range values E[k] whose row position ET[k] is i, in k order.
// The LDS reads are issued in batches of 8 so that they overlap.
template <typename T>
__device__ inline T fold_sum(const int* ET, const T* E, int nextra, int i, T init) {
  T acc = init;
  for (int k0 = 0; k0 < nextra; k0 += 8) {
    int t[8];
    T e[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int kk = min(k0 + k, nextra - 1);
      t[k] = ET[kk];
      e[k] = E[kk];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k0 + k < nextra && t[k] == i) acc += e[k];
  }
  return acc;
}

// Fill the extension margins of an LDS signal buf (index = p - pmin) of length n for
// positions p in [pmin, -1] and [n, pmax].
template <typename T>
__device__ inline void fill_margins(T* buf, int n, int pmin, int pmax, int mode) {
  const int P = mode_period(mode, n);
  const int left = -pmin;                      // positions pmin .. -1
  const int right = pmax >= n ? pmax - n + 1 : 0;
  for (int k = threadIdx.x; k < left + right; k += blockDim.x) {
    const int p = k < left ? pmin + k : n + (k - left);
    bool valid;
    const int i = ext_index(p, n, mode, P, valid);
    buf[p - pmin] = valid ? buf[i - pmin] : T(0);
  }
}

template <typename T>
__device__ inline void load_taps(const T* __restrict__ g0, const T* __restrict__ g1, T* s0,
                                 T* s1, int L, bool reverse) {
  for (int k = threadIdx.x; k < L; k += blockDim.x) {
    const int j = reverse ? L - 1 - k : k;
    s0[k] = g0[j];
    s1[k] = g1[j];
  }
}

// Store VA consecutive outputs o.. of both bands: the high band to global memory, the low
// band to global memory (arow, last level) or to LDS (lds[o]).  Paired stores when the
// caller has established 8-byte alignment (o is even).
template <typename S, typename T>
__device__ inline void store_bands(S* drow, S* arow, T* lds, int o, int no, const T (&y0)[VA],
                                   const T (&y1)[VA], bool vec_g, bool vec_l) {
  static_assert(VA == 2, "paired stores assume two outputs per thread");
  if (o + 1 < no) {
    if constexpr (std::is_same<S, float>::value) {
      if (vec_g) {
        typedef float v2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<v2*>(drow + o) = v2{y1[0], y1[1]};
        if (!lds) *reinterpret_cast<v2*>(arow + o) = v2{y0[0], y0[1]};
      } else {
        drow[o] = y1[0];
        drow[o + 1] = y1[1];
        if (!lds) {
          arow[o] = y0[0];
          arow[o + 1] = y0[1];
        }
      }
    } else {
      Storage<S>::store(drow, o, y1[0]);
      Storage<S>::store(drow, o + 1, y1[1]);
      if (!lds) {
        Storage<S>::store(arow, o, y0[0]);
        Storage<S>::store(arow, o + 1, y0[1]);
      }
    }
    if (lds) {
      if (vec_l) {
        typedef T v2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<v2*>(lds + o) = v2{y0[0], y0[1]};
      } else {
        lds[o] = y0[0];
        lds[o + 1] = y0[1];
      }
    }
  } else if (o < no) {
    Storage<S>::store(drow, o, y1[0]);
    if (lds) lds[o] = y0[0];
    else Storage<S>::store(arow, o, y0[0]);
  }
}

// ------------------------------------------------------------------ analysis chain
// Thread groups per level-0 chunk: 128-thread workgroups (short rows) take a row of up to
// 1280 outputs in one chunk, so all of its loads are in flight at once.
constexpr int achain_groups(int nt) { return nt == 128 ? 5 : GA; }

// One workgroup per row (grid = rows), or, in split mode (levels == 1), `split` chunks of
// CO outputs per workgroup (grid = rows * workgroups_per_row).
template <typename S, typename T, int LT, int NTK>
__global__ void __launch_bounds__(NTK) analysis_chain_kernel(AChainArgs args, int64_t rows,
                                                             int wg_per_row) {
  constexpr int NT = NTK;            // threads per workgroup: 512, or 128 for short rows
  constexpr int GA = achain_groups(NTK);
  constexpr int CO = NT * VA * GA;   // outputs per level-0 chunk
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* const A = reinterpret_cast<T*>(smem_raw);
  T* const B = A + args.capA;
  T* const tap_lds = B + args.capB;  // runtime-length taps (LT == 0)

  const int64_t row = blockIdx.x / wg_per_row;
  const int part = blockIdx.x % wg_per_row;
  const int L = LT > 0 ? LT : args.taps;
  const int off = args.off;
  const int pmin = off - (L - 1);
  const int mode = args.mode;
  const int tid = threadIdx.x;

  const T* gh0 = static_cast<const T*>(args.h0);
  const T* gh1 = static_cast<const T*>(args.h1);
  T hr0r[LT > 0 ? LT : 1], hr1r[LT > 0 ? LT : 1];
  const T* hr0;
  const T* hr1;
  if constexpr (LT > 0) {
#pragma unroll
    for (int i = 0; i < LT; ++i) {
      hr0r[i] = gh0[LT - 1 - i];
      hr1r[i] = gh1[LT - 1 - i];
    }
    hr0 = hr0r;
    hr1 = hr1r;
  } else {
    load_taps(gh0, gh1, tap_lds, tap_lds + L, L, true);
    hr0 = tap_lds;
    hr1 = tap_lds + L;
    __syncthreads();
  }

  // ---- level 0: stream x through the staging window B in chunks of CO outputs
  {
    const int n = args.n_in[0];
    const int no = args.n_out[0];
    const int mode0 = normalize_mode(mode, n);
    const int P = mode_period(mode0, n);
    const S* xrow = static_cast<const S*>(args.x) + row * (int64_t)n;
    S* drow = static_cast<S*>(args.details[0]) + row * (int64_t)no;
    const bool last = args.levels == 1;
    S* arow = last ? static_cast<S*>(args.approx) + row * (int64_t)no : nullptr;

    // paired stores where this row's band starts 8-byte aligned (o is always even)
    const bool vec_g =
        std::is_same<S, float>::value &&
        ((reinterpret_cast<uintptr_t>(drow) | reinterpret_cast<uintptr_t>(arow)) & 7) == 0;
    const bool vec_l = (pmin & 1) == 0;
    const int nchunks = (int)cdiv(no, CO);
    int c_begin = 0, c_end = nchunks;
    if (args.split) {
      c_begin = part * args.split;
      c_end = min(nchunks, c_begin + args.split);
    }
    constexpr int SPAN_MAX = 2 * CO + (LT > 0 ? LT : MAXL_T) - 2;
    constexpr int PF = (SPAN_MAX + NT - 1) / NT;  // prefetch registers (template length)
    // Prefetch registers hold raw samples: the loads are issued here, and the zero padding
    // (a select) and the conversion happen when the chunk is staged, so no wait follows a
    // load where it is issued.  Positions outside the row load the sample their extension
    // maps to (row position 0 under zero padding).
    S pf[PF] = {};

    auto fetch = [&](int c, S (&r)[PF]) {
      const int p0 = 2 * c * CO + pmin;
      const bool interior = p0 >= 0 && p0 + SPAN_MAX <= n;
#pragma unroll
      for (int k = 0; k < PF; ++k) {
        const int idx = tid + k * NT;
        int i = p0 + idx;
        if (idx < SPAN_MAX) {
          if (!interior && (i < 0 || i >= n)) {
            bool valid = true;
            i = ext_index(i, n, mode0, P, valid);
            if (!valid) i = 0;
          }
          r[k] = xrow[i];
        }
      }
    };

    if constexpr (std::is_same<S, float>::value && std::is_same<T, float>::value && LT > 0) {
      // fp32 rows: the window B[idx] = x[p0 + idx] is loaded as 16-byte-aligned groups of four
      // samples, group g holding positions q0 + 4 g + j (q0 = p0 - d aligned down); B has a
      // guard of four elements on either side for the parts of the end groups outside the
      // window.  Only groups lying inside the row [gf, gl] are staged from these loads (every
      // lane loads one, clamped into that range, so each register is written in full and the
      // compiler never waits for it); the window positions outside them -- the extension
      // near the row ends, at most 3 + (L - 1 - off) on the left and 2 L + 6 on the right --
      // are loaded one per thread by the first FX threads at their extension index.
      constexpr int SPAN = 2 * CO + LT - 2;
      constexpr int PW = ((SPAN + 6) / 4 + NT - 1) / NT;
      constexpr int FX = 128;
      typedef float v4f __attribute__((ext_vector_type(4)));
      typedef float v2f __attribute__((ext_vector_type(2)));
      v4u_t w[PW];
      unsigned fx = 0u;
      const unsigned xa = (unsigned)(reinterpret_cast<uintptr_t>(xrow) >> 2);
      const int pmax = 2 * (no - 1) + off;  // last position any output of the level reads
      struct Geo {
        int p0, q0, d, G, gf, gl, nl, r0, nfix;
      };
      auto geom = [&](int c) {
        Geo g;
        g.p0 = 2 * c * CO + pmin;
        g.d = (int)((xa + (unsigned)g.p0) & 3u);
        g.q0 = g.p0 - g.d;
        g.G = (SPAN + g.d + 3) >> 2;
        g.gf = g.q0 >= 0 ? 0 : (3 - g.q0) >> 2;
        g.gl = min(g.G - 1, (n - 4 - g.q0) >> 2);
        const int pend = min(g.p0 + SPAN, pmax + 1);  // window positions read: [p0, pend)
        if (g.gf <= g.gl) {
          g.nl = max(0, min(g.q0 + 4 * g.gf, pend) - g.p0);
          g.r0 = max(g.p0, g.q0 + 4 * (g.gl + 1));
          g.nfix = g.nl + max(0, pend - g.r0);
        } else {
          g.nl = max(0, pend - g.p0);
          g.r0 = pend;
          g.nfix = g.nl;
        }
        g.nfix = min(g.nfix, FX);
        return g;
      };
      auto fetch4 = [&](int c) {
        const Geo g = geom(c);
        if (g.gf <= g.gl) {
#pragma unroll
          for (int k = 0; k < PW; ++k)
            if (k * NT < g.G)
              w[k] = global_load16(xrow + g.q0 + 4 * min(max(tid + k * NT, g.gf), g.gl));
        }
        if (tid < FX && g.nfix > 0) {
          const int t = min(tid, g.nfix - 1);
          const int p = t < g.nl ? g.p0 + t : g.r0 + (t - g.nl);
          int i = min(max(p, 0), n - 1);
          if (p < 0 || p >= n) {
            bool valid = true;
            i = ext_index(p, n, mode0, P, valid);
            if (!valid) i = 0;
          }
          fx = global_load(reinterpret_cast<const unsigned*>(xrow), i);
        }
      };
      auto stage4 = [&](int c) {
        const Geo g = geom(c);
        // every prefetch register counts as used here, on every path, so that the compiler's
        // wait for the loads sits here and not before the next chunk's loads
#pragma unroll
        for (int k = 0; k < PW; ++k) __asm__ volatile("" : : "v"(w[k]));
        __asm__ volatile("" : : "v"(fx));
        if (g.gf <= g.gl) {
#pragma unroll
          for (int k = 0; k < PW; ++k) {
            const int gi = tid + k * NT;
            if (k * NT < g.G && gi >= g.gf && gi <= g.gl) {
              const v4f v = __builtin_bit_cast(v4f, w[k]);
              float* dst = B + 4 * gi - g.d;
              if (g.d == 0) {
                *reinterpret_cast<v4f*>(dst) = v;
              } else if (g.d == 2) {
                *reinterpret_cast<v2f*>(dst) = v2f{v[0], v[1]};
                *reinterpret_cast<v2f*>(dst + 2) = v2f{v[2], v[3]};
              } else {  // d = 1 or 3: dst + 1 is 8-byte aligned
                dst[0] = v[0];
                *reinterpret_cast<v2f*>(dst + 1) = v2f{v[1], v[2]};
                dst[3] = v[3];
              }
            }
          }
        }
        if (tid < g.nfix) {
          const int p = tid < g.nl ? g.p0 + tid : g.r0 + (tid - g.nl);
          const float v = __builtin_bit_cast(float, fx);
          B[p - g.p0] = (mode0 == FDWT_MODE_ZERO && (p < 0 || p >= n)) ? 0.0f : v;
        }
      };
      if (c_begin < c_end) fetch4(c_begin);
      for (int c = c_begin; c < c_end; ++c) {
        __syncthreads();
        stage4(c);
        __syncthreads();
        if (c + 1 < c_end) fetch4(c + 1);
#pragma unroll
        for (int g = 0; g < GA; ++g) {
          const int lo = (g * NT + tid) * VA;  // output offset inside the chunk
          const int o = c * CO + lo;
          if (o >= no) break;
          T y0[VA], y1[VA];
          analysis_pair<T, LT>(B + 2 * lo, hr0, hr1, L, y0, y1);
          store_bands<S, T>(drow, arow, last ? nullptr : A - pmin, o, no, y0, y1, vec_g,
                            vec_l);
        }
      }
    } else if (LT > 0 || L <= MAXL_T) {
      if (c_begin < c_end) fetch(c_begin, pf);
      for (int c = c_begin; c < c_end; ++c) {
        __syncthreads();
        const int p0 = 2 * c * CO + pmin;
#pragma unroll
        for (int k = 0; k < PF; ++k) {
          const int idx = tid + k * NT;
          const int p = p0 + idx;
          if (idx < SPAN_MAX)
            B[idx] = (mode0 == FDWT_MODE_ZERO && (p < 0 || p >= n)) ? T(0)
                                                                  : T(Storage<S>::load(pf + k, 0));
        }
        __syncthreads();
        if (c + 1 < c_end) fetch(c + 1, pf);
#pragma unroll
        for (int g = 0; g < GA; ++g) {
          const int lo = (g * NT + tid) * VA;  // output offset inside the chunk
          const int o = c * CO + lo;
          if (o >= no) break;
          T y0[VA], y1[VA];
          analysis_pair<T, LT>(B + 2 * lo, hr0, hr1, L, y0, y1);
          store_bands<S, T>(drow, arow, last ? nullptr : A - pmin, o, no, y0, y1, vec_g,
                            vec_l);
        }
      }
    } else {
      // long runtime filters: stage without register prefetch (span depends on L)
      const int span_max = 2 * CO + L - 2;
      for (int c = c_begin; c < c_end; ++c) {
        const int p0 = 2 * c * CO + pmin;
        __syncthreads();
        for (int idx = tid; idx < span_max; idx += NT) {
          const int p = p0 + idx;
          bool valid = true;
          const int i = (p >= 0 && p < n) ? p : ext_index(p, n, mode0, P, valid);
          B[idx] = valid ? T(Storage<S>::load(xrow, i)) : T(0);
        }
        __syncthreads();
        for (int g = 0; g < GA; ++g) {
          const int lo = (g * NT + tid) * VA;
          const int o = c * CO + lo;
          if (o >= no) break;
          T y0[VA], y1[VA];
          analysis_pair<T, 0>(B + 2 * lo, hr0, hr1, L, y0, y1);
          for (int q = 0; q < VA; ++q) {
            if (o + q < no) {
              Storage<S>::store(drow, o + q, y1[q]);
              if (last) Storage<S>::store(arow, o + q, y0[q]);
              else A[o + q - pmin] = y0[q];
            }
          }
        }
      }
    }
  }

  // ---- levels 1 .. levels-1: the low band stays in LDS (A -> B -> A ...)
  T* src = A;
  T* dst = B;
  for (int l = 1; l < args.levels; ++l) {
    const int n = args.n_in[l];
    const int no = args.n_out[l];
    const int prev = args.n_out[l - 1];
    // zero tail (waverec trim transpose), then the extension margins
    if (tid == 0 && n > prev) src[prev - pmin] = T(0);
    __syncthreads();
    fill_margins(src, n, pmin, 2 * (no - 1) + off, normalize_mode(mode, n));
    __syncthreads();
    const bool last = l + 1 == args.levels;
    S* drow = static_cast<S*>(args.details[l]) + row * (int64_t)no;
    S* arow = last ? static_cast<S*>(args.approx) + row * (int64_t)no : nullptr;
    // paired stores where this row's band starts 8-byte aligned (o is always even)
    const bool vec_g =
        std::is_same<S, float>::value &&
        ((reinterpret_cast<uintptr_t>(drow) | reinterpret_cast<uintptr_t>(arow)) & 7) == 0;
    const bool vec_l = (pmin & 1) == 0;
    for (int lo = tid * VA; lo < no; lo += NT * VA) {
      T y0[VA], y1[VA];
      analysis_pair<T, LT>(src + 2 * lo, hr0, hr1, L, y0, y1);
      store_bands<S, T>(drow, arow, last ? nullptr : dst - pmin, lo, no, y0, y1, vec_g, vec_l);
    }
    T* t = src;
    src = dst;
    dst = t;
  }
}

// ------------------------------------------------------------------ synthesis chain
// Low band buffers are indexed buf[u + ZL] (ZL = L rounded up to a multiple of 4) with zeros
// for u < 0 and u >= nc.  Per level:
//  1. the few extended positions outside [0, m) are evaluated (E) together with the row
//     position they fold onto (ET), then reduced per edge position (F);
//  2. the row is produced in passes of NT * VS coefficient pairs: the high band of a pass is
//     staged in LDS (D) by coalesced loads, the next pass's prefetched into registers, and
//     each thread computes 2 * VS consecutive positions from two aligned register windows.
template <typename S, typename T, int LT>
__global__ void __launch_bounds__(NT) synthesis_chain_kernel(SChainArgs args, int64_t rows,
                                                             int wg_per_row) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  // per-level parameters, copied from the arguments into LDS once: the level loop reads them
  // with one wave-uniform LDS access instead of a chain of scalar loads at dynamic offsets
  LevelRec* const lrec = reinterpret_cast<LevelRec*>(smem_raw);
  T* const A = reinterpret_cast<T*>(smem_raw + LREC_BYTES);
  T* const B = A + args.capA;
  T* const E = B + args.capB;
  int* const ET = reinterpret_cast<int*>(E + args.capE);
  T* const F = reinterpret_cast<T*>(ET + args.capE);
  T* const D = F + (2 * args.capE + 8);
  T* const tap_lds = D + args.capD;

  const int64_t row = blockIdx.x / wg_per_row;
  const int part = blockIdx.x % wg_per_row;
  const int L = LT > 0 ? LT : args.taps;
  const int H = L / 2;
  const int ZL = (L + 3) & ~3;
  const int off = args.off;
  const int mode = args.mode;
  const int tid = threadIdx.x;

  const T* gh0 = static_cast<const T*>(args.h0);
  const T* gh1 = static_cast<const T*>(args.h1);
  T h0r[LT > 0 ? LT : 1], h1r[LT > 0 ? LT : 1];
  const T* h0;
  const T* h1;
  if constexpr (LT > 0) {
#pragma unroll
    for (int i = 0; i < LT; ++i) {
      h0r[i] = gh0[i];
      h1r[i] = gh1[i];
    }
    h0 = h0r;
    h1 = h1r;
  } else {
    load_taps(gh0, gh1, tap_lds, tap_lds + L, L, false);
    h0 = tap_lds;
    h1 = tap_lds + L;
  }

  // first coefficient pair of a level's passes (aligned to VS): precomputed by the host for
  // whole-row workgroups; split workgroups start at their own window
  auto level_first_pass = [&](int lv) {
    if (!args.split) return args.ub0[lv];
    return ((part * args.split + 1 - off) >> 1) & ~(VS - 1);
  };
  auto drow_of = [&](int lv) -> const S* {
    return args.details[lv] ? static_cast<const S*>(args.details[lv]) + row * (int64_t)args.nc[lv]
                            : nullptr;
  };
  if (tid < args.levels) {
    LevelRec r;
    r.nc = args.nc[tid];
    r.n_out = args.n_out[tid];
    r.ub0 = level_first_pass(tid);
    r.qs0 = args.qs0[tid];
    r.qsn = args.qsn[tid];
    r.qlen = args.qlen[tid];
    r.ncn = tid + 1 < args.levels ? args.nc[tid + 1] : 0;
    r.pad = 0;
    r.drow = drow_of(tid);
    lrec[tid] = r;
  }
  const int dspan = PS + H + 4;
  constexpr int PFD = PS / NT + 1;  // dspan <= PFD * NT since H + 4 <= NT
  // Prefetch registers hold raw coefficients: the loads are issued here and range-masked and
  // converted only when the pass is staged, so no wait follows a load where it is issued.
  // (The load index is clamped into the row; positions outside it are zeroed at staging.)
  S pf[PFD] = {};
  auto fetch_d = [&](const S* dr, int ncl, int pbl) {
    if (!dr) return;
#pragma unroll
    for (int k = 0; k < PFD; ++k) {
      // blocks of NT entirely outside the coefficients are skipped (block-uniform test)
      if (k * NT < dspan && pbl + k * NT < ncl && pbl + k * NT + NT > 0)
        pf[k] = dr[min(max(pbl + tid + k * NT, 0), ncl - 1)];
    }
  };
  // every HBM read the kernel needs for its small levels is issued here, before the low band
  // is staged: the queue (levels 0 .. qlevels - 1) and the first pass of the next level
  S pq[QR] = {};
#pragma unroll
  for (int k = 0; k < QR; ++k) {
    if (k < args.qslots && args.qs_ptr[k]) {
      const int ncl = args.qs_nc[k];
      const S* dr = static_cast<const S*>(args.qs_ptr[k]) + row * (int64_t)ncl;
      pq[k] = dr[min(max(args.qs_u0[k] + tid, 0), ncl - 1)];
    }
  }
  if (args.qlevels < args.levels) {
    const int fl = args.qlevels;
    fetch_d(drow_of(fl), args.nc[fl], level_first_pass(fl));
  }

  // stage the coarsest low band (or, in split mode, this workgroup's window of it)
  int u_lo = 0;
  {
    const int nc = args.nc[0];
    const S* ag = args.approx ? static_cast<const S*>(args.approx) + row * (int64_t)nc : nullptr;
    if (args.split) u_lo = ((((part * args.split) - off) >> 1) - 4) & ~3;
    // whole rows stage the band and the margin that level 0 reads (coefficients up to
    // nc + L + 2 VS + 16); the loads are issued AB at a time so that their latencies overlap
    constexpr int AB = 9;
    const int kend = args.split ? args.capA : min(args.capA, ZL + nc + L + 2 * VS + 16);
    // (raw loads at clamped indices first, range masks and conversions after all of them)
    for (int k0 = tid; k0 < kend; k0 += AB * NT) {
      S v[AB] = {};
      if (ag) {
#pragma unroll
        for (int j = 0; j < AB; ++j) v[j] = ag[min(max(u_lo + k0 + j * NT - ZL, 0), nc - 1)];
      }
#pragma unroll
      for (int j = 0; j < AB; ++j) {
        const int k = k0 + j * NT;
        const int u = u_lo + k - ZL;
        if (k < kend) A[k] = (ag && u >= 0 && u < nc) ? T(Storage<S>::load(v + j, 0)) : T(0);
      }
    }
  }
  __syncthreads();

  T* src = A;
  T* dst = B;
  for (int l = 0; l < args.levels; ++l) {
    const LevelRec lr = load_level(lrec + l);
    const int nc = lr.nc;
    const int m = lr.n_out;
    const bool last = l + 1 == args.levels;
    const S* drow = static_cast<const S*>(lr.drow);
    const T* a0 = src + ZL - u_lo;  // a0[u] = low band coefficient u
    const int md = normalize_mode(mode, m);
    const int P = mode_period(md, m);

    // 1. extended positions outside [0, m) fold back onto row positions near the ends (the
    //    "band").  Whole-row workgroups run their passes over the extended range, park the
    //    out-of-range values (E) and the band values (F) in LDS, and fold them after the
    //    passes; split workgroups evaluate the out-of-range values up front instead.
    const int pmin = off - (L - 1);
    const int pmax = 2 * (nc - 1) + off;
    const int nleft = md == FDWT_MODE_ZERO ? 0 : max(0, -pmin);
    const int nright = md == FDWT_MODE_ZERO ? 0 : max(0, pmax - m + 1);
    const int nextra = nleft + nright;
    const bool inpass = nextra > 0 && !args.split;
    const int band = nextra ? nextra + 2 : 0;  // reflect folds one position further in
    const bool small = m <= 2 * band;
    const int nslot = nextra ? (small ? m : 2 * band) : 0;
    const S* ag = (args.split && args.approx)
                      ? static_cast<const S*>(args.approx) + row * (int64_t)nc : nullptr;

    int i_begin = 0, i_end = m;
    if (args.split) {
      i_begin = part * args.split;
      i_end = min(m, i_begin + args.split);
    }
    const int p_begin = inpass ? min(0, pmin) : i_begin;
    const int p_end = inpass ? max(m, pmax + 1) : i_end;
    const int ub0 = lr.ub0;
    int pb = ub0;
    const bool from_queue = l < args.qlevels;  // this level's d is in the queue

    for (int k = tid; k < nextra; k += NT) {
      const int p = k < nleft ? pmin + k : m + (k - nleft);
      bool valid;
      const int t = ext_index(p, m, md, P, valid);
      ET[k] = valid ? t : -1;
      if (!inpass)
        E[k] = synthesis_point<S, T>(args.split ? nullptr : a0, ag, drow, p, off, nc, h0, h1, L);
    }
    if (!inpass && nextra) {
      __syncthreads();
      for (int sl = tid; sl < nslot; sl += NT) {
        const int i = (small || sl < band) ? sl : m - 2 * band + sl;
        F[sl] = fold_sum(ET, E, nextra, i, T(0));
      }
    }

    // 2. the row, in passes of NT * VS * GS coefficient pairs
    S* orow = last ? static_cast<S*>(args.out) + row * (int64_t)m : nullptr;
    // 16-byte stores when provably aligned: off == 1 puts every thread's first position on
    // a multiple of 4, and m % 4 == 0 keeps rows 16-byte aligned in global memory
    const bool vec_out = std::is_same<S, float>::value && off == 1 && (m % 4) == 0;
    const bool vec_lds = off == 1;
    const int plain_lo = max(i_begin, band);
    const int plain_hi = min(i_end, m - band);
    for (; 2 * pb + off - 1 < p_end; pb += PS) {
      __syncthreads();  // previous pass done with D (F / E / ET written)
      if (from_queue) {
        // a queued level has a single pass, held by queue slots s0 .. s0 + sn - 1
        const int s0 = lr.qs0, sn = lr.qsn, len = lr.qlen;
#pragma unroll
        for (int k = 0; k < QR; ++k) {
          if (k >= s0 && k < s0 + sn) {
            const int idx = (k - s0) * NT + tid;
            const int u = pb + idx;
            if (idx < len)
              D[idx] = (drow && u >= 0 && u < nc) ? T(Storage<S>::load(pq + k, 0)) : T(0);
          }
        }
      } else {
#pragma unroll
        for (int k = 0; k < PFD; ++k) {
          const int idx = tid + k * NT;
          const int u = pb + idx;
          if (idx < dspan)
            D[idx] = (drow && u >= 0 && u < nc) ? T(Storage<S>::load(pf + k, 0)) : T(0);
        }
      }
      __syncthreads();
      const int pn = pb + PS;
      if (!from_queue) {
        if (2 * pn + off - 1 < p_end) {
          fetch_d(drow, nc, pn);
        } else if (!last) {
          // last pass of this level: request the first pass of the next level now
          const LevelRec nr = load_level(lrec + l + 1);
          fetch_d(static_cast<const S*>(nr.drow), nr.nc, nr.ub0);
        }
      }
#pragma unroll
      for (int g = 0; g < GS; ++g) {
        const int lu = (g * NT + tid) * VS;  // coefficient offset inside the pass
        const int ub = pb + lu;
        const int i0 = 2 * ub + off - 1;     // first of this thread's 2 * VS positions
        if (i0 >= p_end) continue;
        T zo[VS], ze[VS];
        synthesis_block<T, LT>(a0 + ub, D + lu, h0, h1, L, zo, ze);
        T v[2 * VS];
#pragma unroll
        for (int q = 0; q < VS; ++q) {
          v[2 * q] = zo[q];
          v[2 * q + 1] = ze[q];
        }
        if (VS == 2 && i0 >= plain_lo && i0 + 2 * VS <= plain_hi && (last ? vec_out : vec_lds)) {
          typedef T v4 __attribute__((ext_vector_type(4)));
          const v4 w = {v[0], v[1], v[2], v[3]};
          if (last) {
            if constexpr (std::is_same<S, float>::value)
              *reinterpret_cast<v4*>(orow + i0) = w;
          } else {
            *reinterpret_cast<v4*>(dst + ZL + i0) = w;
          }
          continue;
        }
        // positions near the row ends (fold band, out-of-range values, partial rows)
#pragma unroll
        for (int j = 0; j < 2 * VS; ++j) {
          const int i = i0 + j;
          T val = v[j];
          if (i >= i_begin && i < i_end) {
            if (band && (i < band || i >= m - band)) {
              const int sl = (small || i < band) ? i : i - (m - 2 * band);
              if (inpass) {
                F[sl] = val;  // folded once every out-of-range value exists
                continue;
              }
              val += F[sl];
            }
            if (last) Storage<S>::store(orow, i, val);
            else dst[ZL + i] = val;
          } else if (inpass) {
            if (i < 0 && i >= pmin) E[i - pmin] = val;
            else if (i >= m && i <= pmax) E[nleft + i - m] = val;
          }
        }
      }
    }
    if (inpass) {
      __syncthreads();
      for (int sl = tid; sl < nslot; sl += NT) {
        const int i = (small || sl < band) ? sl : m - 2 * band + sl;
        const T acc = fold_sum(ET, E, nextra, i, F[sl]);
        if (last) Storage<S>::store(orow, i, acc);
        else dst[ZL + i] = acc;
      }
    }
    __syncthreads();
    if (!last) {
      // zero margins of the next low band (which is the first nc[l+1] outputs)
      // (the next level reads coefficients -ZL .. ncn + L + 2 VS + 8 at most)
      const int ncn = lr.ncn;
      const int cap_dst = (l % 2 == 0) ? args.capB : args.capA;  // dst is B after even levels
      const int zend = min(cap_dst, ZL + ncn + L + 2 * VS + 16);
      for (int k = tid; k < ZL; k += NT) dst[k] = T(0);
      for (int k = ZL + ncn + tid; k < zend; k += NT) dst[k] = T(0);
      __syncthreads();
      T* t = src;
      src = dst;
      dst = t;
    }
  }
}

// Store the 2 VR consecutive values v of positions i0.. of a wave whose lanes hold
// consecutive runs, as 16-byte blocks starting at i0 + sh (16-byte aligned): each lane stores
// v[sh..] and the first sh values of the next lane; lane 0 also stores its first sh values and
// lane 63, whose next lane is in another wave, stores its own values one by one.
template <int SH>
__device__ inline void store_shifted_sh(float* orow, int i0, const float (&v)[2 * VR],
                                        int lane) {
  float nx[SH > 0 ? SH : 1];
#pragma unroll
  for (int j = 0; j < SH; ++j) nx[j] = __shfl_down(v[j], 1);
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < SH; ++j) orow[i0 + j] = v[j];
  }
  if (lane == 63) {
#pragma unroll
    for (int j = SH; j < 2 * VR; ++j) orow[i0 + j] = v[j];
    return;
  }
  float w[2 * VR];
#pragma unroll
  for (int j = 0; j < 2 * VR; ++j) w[j] = j + SH < 2 * VR ? v[j + SH] : nx[j + SH - 2 * VR];
  typedef float v4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int q = 0; q < VR / 2; ++q)
    *reinterpret_cast<v4*>(orow + i0 + SH + 4 * q) =
        v4{w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]};
}

__device__ inline void store_shifted(float* orow, int i0, const float (&v)[2 * VR], int sh,
                                     int lane) {
  if (sh == 1) store_shifted_sh<1>(orow, i0, v, lane);
  else if (sh == 2) store_shifted_sh<2>(orow, i0, v, lane);
  else store_shifted_sh<3>(orow, i0, v, lane);
}

// Sum of the parked values of the extended positions that fold onto row position i (i itself
// included): the positions congruent modulo the period P to i and, for the mirroring
// extensions, to the mirror image of i.  Parked position p sits at E[p - pbeg] below plo and
// at E[(plo - pbeg) + (p - phi)] from phi on.
template <typename T>
__device__ inline T fold_parked(const T* __restrict__ E, int i, int m, int md, int P, int pbeg,
                                int pend, int plo, int phi) {
  auto at = [&](int p) { return E[p < plo ? p - pbeg : (plo - pbeg) + (p - phi)]; };
  T s = at(i);
  int mirror = -1;
  if (md == FDWT_MODE_SYMMETRIC) mirror = P - 1 - i;
  else if (md == FDWT_MODE_REFLECT && i > 0 && i < m - 1) mirror = P - i;
  else if (md == FDWT_MODE_PERIODIZATION && i == m - 1 && P > m) mirror = m;
  // walk each residue class up from its base and down from base - P (no division)
  for (int w = 0; w < 2; ++w) {
    const int base = w == 0 ? i : mirror;
    if (base < 0) continue;
    for (int p = base; p < pend; p += P)
      if (p < 0 || p >= m) s += at(p);
    for (int p = base - P; p >= pbeg; p -= P)
      if (p < pend) s += at(p);
  }
  return s;
}

// Whole-row synthesis chain, persistent: each workgroup reconstructs the rows blockIdx.x,
// blockIdx.x + gridDim.x, .. through all levels (see the plan above).  Per level: the bands
// prefetched for it are staged into LDS and the buffer margins zeroed; each thread computes
// VR consecutive coefficient pairs (2 VR positions) at a time from register windows of both
// bands; positions away from the row ends go straight to the next low band (LDS) or to the
// output row, the others are parked and folded after a barrier by one lane per fold target.
template <typename S, typename T, int LT, bool PRE, int NTK>
__global__ void __launch_bounds__(NTK) synthesis_rows_kernel(SynArgs) {
  constexpr int NT = NTK;  // threads per workgroup: 512, or 128 for short rows
  extern __shared__ __align__(16) unsigned char smem_raw[];
  // the arguments, read in place through the kernel-argument segment pointer: scalar loads at
  // any (wave-uniform) offset, and never a private copy.  (The host compilation pass only
  // type-checks the body; it sees an empty argument block.)
#if defined(__HIP_DEVICE_COMPILE__)
  typedef __attribute__((address_space(4))) const SynArgs KArgs;
  KArgs& args = *(KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
#else
  const SynArgs args{};
#endif
  SynTab* const tab = reinterpret_cast<SynTab*>(smem_raw);
  T* const lds = reinterpret_cast<T*>(smem_raw + sizeof(SynTab));
  const int J = args.levels;
  const int L = LT > 0 ? LT : args.taps;
  const int ZL = (L + 3) & ~3;
  const int off = args.off;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int64_t rows = args.rows;

  const T* gh0 = static_cast<const T*>(args.h0);
  const T* gh1 = static_cast<const T*>(args.h1);
  T h0r[LT > 0 ? LT : 1], h1r[LT > 0 ? LT : 1];
  const T* h0;
  const T* h1;
  if constexpr (LT > 0) {
#pragma unroll
    for (int i = 0; i < LT; ++i) {
      h0r[i] = gh0[i];
      h1r[i] = gh1[i];
    }
    h0 = h0r;
    h1 = h1r;
  } else {
    load_taps(gh0, gh1, lds + args.offTap, lds + args.offTap + L, L, false);
    h0 = lds + args.offTap;
    h1 = lds + args.offTap + L;
  }
  {
    typedef int v4i __attribute__((ext_vector_type(4)));
#if defined(__HIP_DEVICE_COMPILE__)
    typedef __attribute__((address_space(4))) const v4i KWord;
#else
    typedef const v4i KWord;
#endif
    KWord* src = reinterpret_cast<KWord*>(&args.tab);
    v4i* dst = reinterpret_cast<v4i*>(tab);
    for (int k = tid; k < (int)(sizeof(SynTab) / 16); k += NT) dst[k] = src[k];
  }
  __syncthreads();

  // ---- prefetch registers: raw band values, converted only when staged
  constexpr int NPA = syn_pa((int)sizeof(S));
  S pa[NPA][PQ], pb[PB][PQ];
#pragma unroll
  for (int k = 0; k < NPA; ++k)
#pragma unroll
    for (int j = 0; j < PQ; ++j) pa[k][j] = S{};
#pragma unroll
  for (int k = 0; k < PB; ++k)
#pragma unroll
    for (int j = 0; j < PQ; ++j) pb[k][j] = S{};
  const int voff = tid * (int)sizeof(S);  // this lane's byte offset in a register's first NT
  // Load descriptors and staging words come from the LDS copy of the tables (every lane reads
  // the same address) and are made wave-uniform, so the row address and the buffer range are
  // scalar arithmetic; the loads take voff plus a constant per j.
  auto issue = [&](auto& regs, const SynLoad* t, int n, int64_t r) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < n; ++k) {
      const SynLoad d = lds_uniform(t + k);
      if (d.cnt > 0) {
        char* base = const_cast<char*>(static_cast<const char*>(d.base)) + r * (int64_t)d.stride;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            base, (short)0, d.cnt * (int)sizeof(S), 0x00020000);
#pragma unroll
        for (int j = 0; j < PQ; ++j)
          regs[k][j] = buffer_load_raw<S>(rs, voff, j * NT * (int)sizeof(S));
      }
    }
  };
  auto stage = [&](auto& regs, const uint32_t* t, int n, uint32_t mask) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < n; ++k) {
      if (mask & (1u << k)) {
        const uint32_t w = (uint32_t)__builtin_amdgcn_readfirstlane(t[k]);
        const int dest = (int)(w & 0x3ffffu), cnt = (int)(w >> 18);
        T* const d = lds + dest + tid;
#pragma unroll
        for (int j = 0; j < PQ; ++j)
          if (tid + j * NT < cnt) d[j * NT] = T(Storage<S>::load(&regs[k][j], 0));
      }
    }
  };
  auto issue_head = [&](int64_t r) __attribute__((always_inline)) { issue(pa, tab->ldA, NPA, r); };
  auto issue_tail = [&](int64_t r) __attribute__((always_inline)) { issue(pb, tab->ldB, PB, r); };
  auto stage_head = [&](int l) __attribute__((always_inline)) {
    stage(pa, tab->stA, NPA, (uint32_t)__builtin_amdgcn_readfirstlane(tab->maskA[l]));
  };
  auto stage_tail = [&]() __attribute__((always_inline)) {
    stage(pb, tab->stB, PB, (1u << PB) - 1u);
  };
  auto wait_loads = [&]() __attribute__((always_inline)) { __builtin_amdgcn_s_waitcnt(0x0F70); };  // vmcnt(0)
  // without prefetch: the bands of level l, NT * PB * PQ coefficients at a time through pb
  auto direct = [&](int l, int64_t r) __attribute__((always_inline)) {
    const int src = __builtin_amdgcn_readfirstlane(tab->lv[l].src);
    const int dbuf = __builtin_amdgcn_readfirstlane(tab->lv[l].dbuf);
    for (int s = 0; s < 2; ++s) {
      if (s == 0 && l > 0) continue;  // a_0 belongs to level 0 only
      const S* band = static_cast<const S*>(args.band[s == 0 ? 0 : l + 1]);
      if (!band) continue;
      const int cnt = args.nc[l];
      T* dstp = lds + (s == 0 ? src : dbuf) + ZL;
      for (int c0 = 0; c0 < cnt; c0 += NT * PB * PQ) {
#pragma unroll
        for (int k = 0; k < PB * PQ; ++k) {
          const int c = c0 + k * NT + tid;
          if (c0 + k * NT < cnt)
            pb[k / PQ][k % PQ] = global_load(band, r * (int64_t)cnt + (c < cnt ? c : cnt - 1));
        }
        wait_loads();
#pragma unroll
        for (int k = 0; k < PB * PQ; ++k) {
          const int c = c0 + k * NT + tid;
          if (c < cnt) dstp[c] = T(Storage<S>::load(&pb[k / PQ][k % PQ], 0));
        }
      }
    }
  };
  auto zero = [&](int a, int b) __attribute__((always_inline)) {
    for (int k = a + tid; k < b; k += NT) lds[k] = T(0);
  };

  const bool vec_lds = ((off - 1) & 3) == 0;  // a thread's first position is a multiple of 4
  const int sh = (4 - ((off - 1) & 3)) & 3;    // else its distance to the next multiple of 4

  // one level: margins, main pass, fold (the bands are staged)
  // (always inlined: an outlined lambda would take the address of the kernel arguments, which
  // then get copied to private memory)
  auto level = [&](int l, int64_t row) __attribute__((always_inline)) {
    const SynLevel lv = lds_uniform(tab->lv + l);
    const bool last = l + 1 == J;
    // zero margins of both bands (and the whole band when it is absent)
    zero(lv.src, lv.src + ZL);
    zero(lv.src + ZL + lv.nva, lv.src + ZL + lv.zhi);
    zero(lv.dbuf, lv.dbuf + ZL);
    zero(lv.dbuf + ZL + lv.nvd, lv.dbuf + ZL + lv.zhi);
    __syncthreads();

    // main pass
    const int m = lv.m;
    const T* a0 = lds + lv.src + ZL;   // a0[v] = low band coefficient v
    const T* dp = lds + lv.dbuf + ZL;  // dp[v] = high band coefficient v
    T* const E = lds + args.offE;
    T* const dst = last ? nullptr : lds + lv.dst + ZL;
    S* const orow = last ? static_cast<S*>(args.out) + row * (int64_t)m : nullptr;
    // output rows: the shift to the next 16-byte boundary follows from the row's own address
    // (rows of any length), LDS bands from the offset alone
    const int osh = last ? (int)((4u - (((unsigned)(reinterpret_cast<uintptr_t>(orow) >> 2) +
                                          (unsigned)(off - 1)) & 3u)) & 3u)
                         : sh;
    const bool vec_out = std::is_same<S, float>::value && osh == 0;
    const bool vec_shift = std::is_same<S, float>::value && osh != 0;
    const int plo = lv.plo, phi = lv.phi, pbeg = lv.pbeg, pend = lv.pend;
    // VV consecutive pairs from v0 (vw: the first pair of the thread's wave, VV == VR only)
    auto pairs = [&](auto vv, int v0, int vw) __attribute__((always_inline)) {
      constexpr int VV = decltype(vv)::value;
      T zo[VV], ze[VV];
      synthesis_block<T, LT, VV>(a0 + v0, dp + v0, h0, h1, L, zo, ze);
      T v[2 * VV];
#pragma unroll
      for (int q = 0; q < VV; ++q) {
        v[2 * q] = zo[q];
        v[2 * q + 1] = ze[q];
      }
      const int i0 = 2 * v0 + off - 1;  // first of this thread's 2 VV positions
      if constexpr (VV == VR && std::is_same<S, float>::value) {
        // whole waves inside the plain range of the output row: shifted 16-byte stores
        const int iw = 2 * vw + off - 1;
        if (last && vec_shift && iw >= plo && iw + 128 * VR <= phi) {
          store_shifted(orow, i0, v, osh, lane);
          return;
        }
      }
      if constexpr (VV == VR) {
        if (i0 >= plo && i0 + 2 * VR <= phi && (last ? vec_out : vec_lds)) {
          typedef T v4 __attribute__((ext_vector_type(4)));
#pragma unroll
          for (int q = 0; q < VR / 2; ++q) {
            const v4 w = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
            if (last) {
              if constexpr (std::is_same<S, float>::value)
                *reinterpret_cast<v4*>(orow + i0 + 4 * q) = w;
            } else {
              *reinterpret_cast<v4*>(dst + i0 + 4 * q) = w;
            }
          }
          return;
        }
      }
#pragma unroll
      for (int j = 0; j < 2 * VV; ++j) {
        const int p = i0 + j;
        if (p >= plo && p < phi) {
          if (last) Storage<S>::store(orow, p, v[j]);
          else dst[p] = v[j];
        } else if (p >= pbeg && p < pend) {
          E[p < plo ? p - pbeg : (plo - pbeg) + (p - phi)] = v[j];
        }
      }
    };
    // whole passes of NT VR pairs, then the level's remainder one pair per thread: a pass
    // costs the same with a few pairs as with all, and the remainder (a few dozen pairs on
    // the long levels, the whole of the short ones) is on every level's critical path
    const int vmid = lv.vbeg + (lv.vend - lv.vbeg) / (NT * VR) * (NT * VR);
    for (int vw = lv.vbeg + (tid - lane) * VR; vw < vmid; vw += NT * VR)
      pairs(std::integral_constant<int, VR>{}, vw + lane * VR, vw);
    for (int v0 = vmid + tid; v0 < lv.vend; v0 += NT) pairs(std::integral_constant<int, 1>{}, v0, 0);
    __syncthreads();

    // fold targets near the row ends (none in zero mode); the next level's staging (other
    // LDS regions) may run meanwhile
    const int nl = plo < lv.mw ? plo : lv.mw;
    for (int t = tid; t < lv.nt; t += NT) {
      const int i = t < nl ? t : phi + (t - nl);
      const T s = fold_parked(E, i, m, lv.md, lv.P, pbeg, pend, plo, phi);
      if (last) Storage<S>::store(orow, i, s);
      else dst[i] = s;
    }
  };

  // (one schedule for every row, with unconditional loads: a load issued on some paths only
  // would make the compiler copy the prefetch registers between paths, and every copy of a
  // register whose load is in flight waits for all loads)
  int64_t row = blockIdx.x;
  if constexpr (PRE) issue_head(row);
  for (; row < rows; row += gridDim.x) {
    const int64_t next = row + gridDim.x < rows ? row + gridDim.x : rows - 1;
    if constexpr (PRE) {
      // levels 0 .. J-2: the head (requested before the previous row's last level) is
      // complete after this wait; this row's tail is requested here, waited for at level J-1
      wait_loads();
      stage_head(0);
      issue_tail(row);
    } else {
      direct(0, row);
    }
    for (int l = 0; l + 1 < J; ++l) {
      if (l > 0) {
        if constexpr (PRE) stage_head(l);
        else direct(l, row);
      }
      level(l, row);
    }
    // level J-1: the tail; the next row's head is requested before the main pass, whose
    // duration covers its latency
    if constexpr (PRE) {
      wait_loads();
      stage_tail();
      issue_head(next);
    } else if (J > 1) {
      direct(J - 1, row);
    }
    level(J - 1, row);
  }
}

// ------------------------------------------------------------------ host side
template <typename S>
struct Dispatch;

inline bool fits_lds(int64_t bytes) { return bytes <= 160 * 1024; }

// Raise the dynamic LDS limit of a kernel to the full 160 KiB.  Called once per kernel
// instantiation through a function-local static of the (templated) launcher.
template <typename K>
inline bool allow_full_lds(K kernel) {
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  return true;
}

template <typename S, typename T, int LT>
int launch_achain(const AChainArgs& a, int64_t rows, int wg_per_row, size_t lds, int nt,
                  hipStream_t st) {
  auto k = nt == 128 ? analysis_chain_kernel<S, T, LT, 128> : analysis_chain_kernel<S, T, LT, 512>;
  static const bool lds_ok =
      allow_full_lds(analysis_chain_kernel<S, T, LT, 128>) &&
      allow_full_lds(analysis_chain_kernel<S, T, LT, 512>);
  (void)lds_ok;
  hipLaunchKernelGGL(k, dim3((unsigned)(rows * wg_per_row)), dim3(nt), lds, st, a, rows,
                     wg_per_row);
  FDWT_CHECK_LAUNCH();
  return 0;
}

template <typename S, typename T, int LT>
int launch_schain(const SChainArgs& a, int64_t rows, int wg_per_row, size_t lds,
                  hipStream_t st) {
  auto k = synthesis_chain_kernel<S, T, LT>;
  static const bool lds_ok = allow_full_lds(k);
  (void)lds_ok;
  hipLaunchKernelGGL(k, dim3((unsigned)(rows * wg_per_row)), dim3(NT), lds, st, a, rows,
                     wg_per_row);
  FDWT_CHECK_LAUNCH();
  return 0;
}

// Compute units of the current device, cached per device.  The cache entries are atomics:
// concurrent first calls from several host threads may each query the device, and they all
// store the same value.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Workgroups of a persistent whole-row kernel: as many as fit on the device at once (by its
// occupancy at this LDS size), then evened out so that every workgroup gets the same number
// of rows (the last one possibly fewer).
template <typename K>
inline int64_t persistent_grid(K kernel, int nt, size_t lds, int64_t rows) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel),
                                                   nt, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int64_t full = (int64_t)per_cu * device_cus();
  if (rows <= full) return rows;
  const int64_t per_wg = cdiv(rows, full);
  return cdiv(rows, per_wg);
}

template <typename S, typename T, int LT>
int launch_rchain(const SynArgs& a, size_t lds, int nt, hipStream_t st) {
  static const bool lds_ok = allow_full_lds(synthesis_rows_kernel<S, T, LT, true, 512>) &&
                             allow_full_lds(synthesis_rows_kernel<S, T, LT, false, 512>) &&
                             allow_full_lds(synthesis_rows_kernel<S, T, LT, true, 128>) &&
                             allow_full_lds(synthesis_rows_kernel<S, T, LT, false, 128>);
  (void)lds_ok;
  auto k = nt == 128 ? (a.prefetch ? synthesis_rows_kernel<S, T, LT, true, 128>
                                   : synthesis_rows_kernel<S, T, LT, false, 128>)
                     : (a.prefetch ? synthesis_rows_kernel<S, T, LT, true, 512>
                                   : synthesis_rows_kernel<S, T, LT, false, 512>);
  const int64_t grid = persistent_grid(k, nt, lds, a.rows);
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(nt), lds, st, a);
  FDWT_CHECK_LAUNCH();
  return 0;
}

#define FDWT_TAPS_SWITCH(L, FN, ...)                                                     \
  switch (L) {                                                                           \
    case 2: return FN<S, float, 2>(__VA_ARGS__);                                         \
    case 4: return FN<S, float, 4>(__VA_ARGS__);                                         \
    case 6: return FN<S, float, 6>(__VA_ARGS__);                                         \
    case 8: return FN<S, float, 8>(__VA_ARGS__);                                         \
    case 10: return FN<S, float, 10>(__VA_ARGS__);                                       \
    case 12: return FN<S, float, 12>(__VA_ARGS__);                                       \
    case 14: return FN<S, float, 14>(__VA_ARGS__);                                       \
    case 16: return FN<S, float, 16>(__VA_ARGS__);                                       \
    case 18: return FN<S, float, 18>(__VA_ARGS__);                                       \
    case 20: return FN<S, float, 20>(__VA_ARGS__);                                       \
    case 22: return FN<S, float, 22>(__VA_ARGS__);                                       \
    case 24: return FN<S, float, 24>(__VA_ARGS__);                                       \
    case 26: return FN<S, float, 26>(__VA_ARGS__);                                       \
    case 28: return FN<S, float, 28>(__VA_ARGS__);                                       \
    case 30: return FN<S, float, 30>(__VA_ARGS__);                                       \
    case 32: return FN<S, float, 32>(__VA_ARGS__);                                       \
    default: return FN<S, float, 0>(__VA_ARGS__);                                        \
  }

template <typename S>
int run_achain(const AChainArgs& a, int64_t rows, int wg, size_t lds, int nt, hipStream_t st,
               bool templated) {
  if (templated) { FDWT_TAPS_SWITCH(a.taps, launch_achain, a, rows, wg, lds, nt, st) }
  return launch_achain<S, float, 0>(a, rows, wg, lds, nt, st);
}

template <typename S>
int run_schain(const SChainArgs& a, int64_t rows, int wg, size_t lds, hipStream_t st,
               bool templated) {
  if (templated) { FDWT_TAPS_SWITCH(a.taps, launch_schain, a, rows, wg, lds, st) }
  return launch_schain<S, float, 0>(a, rows, wg, lds, st);
}

template <typename S>
int run_rchain(const SynArgs& a, size_t lds, int nt, hipStream_t st, bool templated) {
  if (templated) { FDWT_TAPS_SWITCH(a.taps, launch_rchain, a, lds, nt, st) }
  return launch_rchain<S, float, 0>(a, lds, nt, st);
}

int dispatch_rchain(const SynArgs& a, size_t lds, int nt, int dtype, hipStream_t st) {
  const bool templ = a.taps <= MAXL_T;
  switch (dtype) {
    case FDWT_F32: return run_rchain<float>(a, lds, nt, st, templ);
    case FDWT_F16: return run_rchain<__half>(a, lds, nt, st, templ);
    case FDWT_BF16: return run_rchain<bf16_t>(a, lds, nt, st, templ);
    case FDWT_F64: return launch_rchain<double, double, 0>(a, lds, nt, st);
    default: return FDWT_ERR_ARG;
  }
}

int dispatch_achain(const AChainArgs& a, int64_t rows, int wg, size_t lds, int nt, int dtype,
                    hipStream_t st) {
  const bool templ = a.taps <= MAXL_T;
  switch (dtype) {
    case FDWT_F32: return run_achain<float>(a, rows, wg, lds, nt, st, templ);
    case FDWT_F16: return run_achain<__half>(a, rows, wg, lds, nt, st, templ);
    case FDWT_BF16: return run_achain<bf16_t>(a, rows, wg, lds, nt, st, templ);
    case FDWT_F64: return launch_achain<double, double, 0>(a, rows, wg, lds, nt, st);
    default: return FDWT_ERR_ARG;
  }
}

int dispatch_schain(const SChainArgs& a, int64_t rows, int wg, size_t lds, int dtype,
                    hipStream_t st) {
  const bool templ = a.taps <= MAXL_T;
  switch (dtype) {
    case FDWT_F32: return run_schain<float>(a, rows, wg, lds, st, templ);
    case FDWT_F16: return run_schain<__half>(a, rows, wg, lds, st, templ);
    case FDWT_BF16: return run_schain<bf16_t>(a, rows, wg, lds, st, templ);
    case FDWT_F64: return launch_schain<double, double, 0>(a, rows, wg, lds, st);
    default: return FDWT_ERR_ARG;
  }
}

inline int compute_size(int dtype) { return dtype == FDWT_F64 ? 8 : 4; }

inline bool valid_common(int64_t rows, int taps, int mode, int dtype) {
  return rows >= 0 && taps >= 2 && taps % 2 == 0 && taps <= MAX_TAPS && mode >= 0 && mode <= 4 &&
         dtype >= 0 && dtype <= 3;
}

// LDS layout of an analysis chain: A holds the inputs of odd levels, B the staging window of
// level 0 and the inputs of even levels >= 2; sizes in compute elements.
void achain_caps(const int64_t* n_in, const int64_t* n_out, int levels, int L, int co,
                 int* capA, int* capB) {
  // the level-0 window (chunks of co outputs) is staged in aligned groups of four: up to
  // three elements before B (the last four elements of A are a guard) and three after it
  const int64_t stage = 2 * (int64_t)co + (L > MAXL_T ? L : MAXL_T) - 2 + 4;
  int64_t a = 0, b = stage;
  for (int l = 1; l < levels; ++l) {
    const int64_t need = std::max<int64_t>(2 * n_out[l] + L, n_in[l] + L) + 2;
    if (l % 2) a = std::max(a, need);
    else b = std::max(b, need);
  }
  a += 4;
  *capA = (int)((a + 3) & ~3);
  *capB = (int)((b + 3) & ~3);
}

int extras_count(int64_t nc, int64_t m, int L, int off, int mode) {
  if (normalize_mode(mode, (int)m) == FDWT_MODE_ZERO) return 0;
  const int64_t pmin = off - (L - 1);
  const int64_t pmax = 2 * (nc - 1) + off;
  return (int)(std::max<int64_t>(0, -pmin) + std::max<int64_t>(0, pmax - m + 1));
}

void schain_caps(const int64_t* nc, const int64_t* n_out, int levels, int L, int off, int mode,
                 int split, int* capA, int* capB, int* capE, int* capD) {
  const int64_t zl = (L + 3) & ~3;
  const int64_t margin = zl + L + 2 * VS + 24;
  int64_t a, b = 0, e = 4;
  if (split) a = split / 2 + margin + 16;
  else a = nc[0] + margin;
  for (int l = 0; l < levels; ++l) {
    e = std::max<int64_t>(e, extras_count(nc[l], n_out[l], L, off, mode));
    if (l + 1 == levels) break;
    const int64_t need = n_out[l] + margin;  // output of level l = low band of level l + 1
    if (l % 2 == 0) b = std::max(b, need);
    else a = std::max(a, need);
  }
  *capA = (int)((a + 3) & ~3);
  *capB = (int)((b + 3) & ~3);
  *capE = (int)((e + 3) & ~3);
  *capD = (int)((PS + L / 2 + 8 + 3) & ~3);
}

}  // namespace
}  // namespace fdwt

using namespace fdwt;

extern "C" int64_t fdwt_chain_max_length(int32_t taps, int32_t dtype) {
  // analysis: A ~ n/2 + 2L, B ~ max(stage, n/4 + 2L); synthesis: similar.  Keep <= 160 KiB.
  const int64_t budget =
      (160 * 1024 - LREC_BYTES) / compute_size(dtype) - 4 * (int64_t)taps - 4 * MAXL_T - 64;
  const int64_t stage = 2 * (int64_t)CO + MAXL_T;
  // n/2 + max(stage, n/4) + 6L <= budget
  int64_t n = 2 * (budget - stage - 6 * (int64_t)taps);
  const int64_t n2 = (budget - 6 * (int64_t)taps) * 4 / 3;
  if (n2 / 4 > stage) n = n2;  // the n/4 term dominates the staging window
  // synthesis (whole-row kernel): tables (< 8 KiB) + P ~ n/2, Q + D ~ n/2 (the last level's
  // two bands), each with margins of about 2L + 16, the parked fold values (< 4L + 8) and the
  // taps: n + 12 L + 80 elements at most
  const int64_t ns = (160 * 1024 - 8192) / compute_size(dtype) - 12 * (int64_t)taps - 96;
  if (ns < n) n = ns;
  return n > 0 ? n : 0;
}

extern "C" int fdwt_analysis_chain(const void* x, void* const* details, void* approx,
                                   const void* h0, const void* h1, int64_t rows,
                                   const int64_t* n_in, const int64_t* n_out, int32_t levels,
                                   int32_t taps, int32_t mode, int32_t off, int32_t dtype,
                                   void* stream) {
  if (!valid_common(rows, taps, mode, dtype) || levels < 1 || levels > FDWT_MAX_LEVELS ||
      !n_in || !n_out)
    return FDWT_ERR_ARG;
  if (rows == 0) return 0;
  AChainArgs a{};
  for (int l = 0; l < levels; ++l) {
    if (n_in[l] < 1 || n_out[l] < 1 || n_in[l] > INT32_MAX / 2 || n_out[l] > INT32_MAX / 4)
      return FDWT_ERR_ARG;
    if (l > 0 && (n_in[l] < n_out[l - 1] || n_in[l] > n_out[l - 1] + 1)) return FDWT_ERR_ARG;
    if (!details || !details[l]) return FDWT_ERR_ARG;
    a.details[l] = details[l];
    a.n_in[l] = (int32_t)n_in[l];
    a.n_out[l] = (int32_t)n_out[l];
  }
  if (!x || !approx || !h0 || !h1) return FDWT_ERR_ARG;
  // the extension must stay within one row period of the signal's support: guaranteed by
  // n_out <= (n + L - 1) / 2 + 1 for every mode
  for (int l = 0; l < levels; ++l)
    if (2 * (n_out[l] - 1) + off > n_in[l] + 2 * (int64_t)taps + 2) return FDWT_ERR_ARG;
  a.x = x;
  a.approx = approx;
  a.h0 = h0;
  a.h1 = h1;
  a.levels = levels;
  a.taps = taps;
  a.mode = mode;  // normalised per level in the kernel (reflect on one sample)
  a.off = off;
  if (off < 0 || off > taps) return FDWT_ERR_ARG;
  // short rows: 128-thread workgroups (one chunk of up to 1280 outputs) keep the threads
  // busy and let four times as many rows share a CU
  const int nt = n_out[0] <= 3 * 128 * VA * GA ? 128 : NT;
  const int co = nt * VA * achain_groups(nt);
  int capA, capB;
  achain_caps(n_in, n_out, levels, taps, co, &capA, &capB);
  a.capA = capA;
  a.capB = capB;
  const int cs = compute_size(dtype);
  const size_t lds = (size_t)(capA + capB + 2 * taps + 4) * cs;
  if (!fits_lds((int64_t)lds)) return FDWT_ERR_TOO_LONG;
  int wg = 1;
  a.split = 0;
  const int64_t nchunks = cdiv(n_out[0], co);
  if (levels == 1 && rows < 1024 && nchunks > 1) {
    // few long rows: spread the chunks of a row over several workgroups
    const int64_t want = cdiv(2048, rows);
    a.split = (int)std::max<int64_t>(1, cdiv(nchunks, want));
    wg = (int)cdiv(nchunks, a.split);
  }
  // a launch holds at most 2^32 - 1 threads: larger batches run as consecutive launches over
  // row ranges (the row pointers offset accordingly)
  const int64_t per = std::max<int64_t>(1, (int64_t)(0xffffffffu / (unsigned)nt) / wg);
  const int es = dtype_size(dtype);
  for (int64_t r0 = 0; r0 < rows; r0 += per) {
    AChainArgs c = a;
    c.x = static_cast<const char*>(a.x) + r0 * n_in[0] * es;
    for (int l = 0; l < levels; ++l) c.details[l] = static_cast<char*>(a.details[l]) + r0 * n_out[l] * es;
    c.approx = static_cast<char*>(a.approx) + r0 * n_out[levels - 1] * es;
    const int rc = dispatch_achain(c, std::min(per, rows - r0), wg, lds, nt, dtype,
                                   static_cast<hipStream_t>(stream));
    if (rc) return rc;
  }
  return 0;
}

// Whole-row synthesis chain: LDS layout, level records and prefetch jobs, launch.
// Returns FDWT_ERR_TOO_LONG when a row does not fit in 160 KiB of LDS.
int synthesis_rows(const SChainArgs& s, int64_t rows, int dtype, hipStream_t st) {
  const int J = s.levels, L = s.taps;
  if (J > FDWT_SYN_MAX_LEVELS) return FDWT_ERR_ARG;
  const int ZL = (L + 3) & ~3;
  const int cs = compute_size(dtype);
  SynGeom geo[FDWT_SYN_MAX_LEVELS];
  int64_t capP = 0, capQ = 0, capD = 0, capE = 4;
  int64_t need_last = 0;
  for (int l = 0; l < J; ++l) {
    const bool last = l + 1 == J;
    geo[l] = syn_geom(s.nc[l], s.n_out[l], last ? 0 : s.nc[l + 1], last, L, s.off, s.mode);
    const int64_t need = ZL + (int64_t)geo[l].zhi;  // coefficients -ZL .. zhi of either band
    if (((J - 1 - l) & 1) == 0) capP = std::max(capP, need);
    else capQ = std::max(capQ, need);
    if (last) need_last = need;
    else capD = std::max(capD, need);
    capE = std::max<int64_t>(capE, geo[l].ne);
  }
  capD = std::max(capD, need_last - capQ);  // the last level's high band spans Q and D
  auto r4 = [](int64_t v) { return (v + 3) & ~(int64_t)3; };
  const int64_t yP = 0, yQ = r4(capP), yD = yQ + r4(capQ), yE = yD + r4(capD);
  const int64_t yT = yE + r4(capE);
  const size_t lds = sizeof(SynTab) + (size_t)(yT + r4(2 * L)) * cs;
  if (!fits_lds((int64_t)lds)) return FDWT_ERR_TOO_LONG;

  SynArgs a{};
  a.band[0] = s.approx;
  for (int l = 0; l < J; ++l) {
    a.band[l + 1] = s.details[l];
    a.nc[l] = s.nc[l];
    const SynGeom& g = geo[l];
    SynLevel& r = a.tab.lv[l];
    r.m = g.m;
    r.mw = g.mw;
    r.md = g.md;
    r.P = g.P;
    r.pbeg = g.pbeg;
    r.pend = g.pend;
    r.plo = g.plo;
    r.phi = g.phi;
    r.vbeg = g.vbeg;
    r.vend = g.vend;
    r.zhi = g.zhi;
    r.nt = g.nt;
    r.src = syn_src(l, J, (int)yP, (int)yQ);
    r.dst = l + 1 == J ? -1 : syn_src(l + 1, J, (int)yP, (int)yQ);
    r.dbuf = syn_dbuf(l, J, (int)yQ, (int)yD);
    r.nva = l > 0 ? s.nc[l] : (s.approx ? s.nc[0] : 0);
    r.nvd = s.details[l] ? s.nc[l] : 0;
  }
  // threads per workgroup: 128 for short rows (the last level's pairs in at most three passes
  // of 128 threads), else 512
  const int nt = geo[J - 1].vend - geo[J - 1].vbeg <= 3 * 128 * VR ? 128 : 512;
  const bool pre = syn_regs(
      J, s.nc, s.approx, s.details, ZL, (int)yP, (int)yQ, (int)yD, PQ * nt,
      syn_pa(dtype_size(dtype)), PB,
      [&](bool tail, int k, int c0, int cnt, int dest, int l, bool is_approx) {
        const void* band = is_approx ? s.approx : s.details[l];
        const int es = dtype_size(dtype);
        const SynLoad ld{static_cast<const char*>(band) + (size_t)c0 * es, s.nc[l] * es, cnt};
        if (tail) {
          a.tab.ldB[k] = ld;
          a.tab.stB[k] = syn_stage_word(dest, cnt);
        } else {
          a.tab.ldA[k] = ld;
          a.tab.stA[k] = syn_stage_word(dest, cnt);
          a.tab.maskA[l] |= 1u << k;
        }
      });
  if (!pre) {  // no prefetch: clear whatever was filled before the overflow
    for (int k = 0; k < PA; ++k) a.tab.ldA[k] = SynLoad{nullptr, 0, 0}, a.tab.stA[k] = 0;
    for (int k = 0; k < PB; ++k) a.tab.ldB[k] = SynLoad{nullptr, 0, 0}, a.tab.stB[k] = 0;
    for (int l = 0; l < J; ++l) a.tab.maskA[l] = 0;
  }
  a.out = s.out;
  a.h0 = s.h0;
  a.h1 = s.h1;
  a.rows = rows;
  a.levels = J;
  a.taps = L;
  a.off = s.off;
  a.prefetch = pre ? 1 : 0;
  a.offE = (int32_t)yE;
  a.offTap = (int32_t)yT;
  return dispatch_rchain(a, lds, nt, dtype, st);
}

extern "C" int fdwt_synthesis_chain(const void* approx, const void* const* details, void* out,
                                    const void* h0, const void* h1, int64_t rows,
                                    const int64_t* nc, const int64_t* n_out, int32_t levels,
                                    int32_t taps, int32_t mode, int32_t off, int32_t dtype,
                                    void* stream) {
  if (!valid_common(rows, taps, mode, dtype) || levels < 1 || levels > FDWT_MAX_LEVELS ||
      !nc || !n_out || !out || !h0 || !h1)
    return FDWT_ERR_ARG;
  if (rows == 0) return 0;
  SChainArgs a{};
  for (int l = 0; l < levels; ++l) {
    if (nc[l] < 1 || n_out[l] < 1 || nc[l] > INT32_MAX / 4 || n_out[l] > INT32_MAX / 2)
      return FDWT_ERR_ARG;
    if (l > 0 && (nc[l] > n_out[l - 1] || nc[l] < n_out[l - 1] - 1)) return FDWT_ERR_ARG;
    // every output position must be reachable by the coefficients' taps
    if (n_out[l] > 2 * nc[l] + 2) return FDWT_ERR_ARG;
    a.details[l] = details ? details[l] : nullptr;
    a.nc[l] = (int32_t)nc[l];
    a.n_out[l] = (int32_t)n_out[l];
  }
  if (off < 0 || off > taps) return FDWT_ERR_ARG;
  a.approx = approx;
  a.out = out;
  a.h0 = h0;
  a.h1 = h1;
  a.levels = levels;
  a.taps = taps;
  a.mode = mode;
  a.off = off;
  int wg = 1;
  a.split = 0;
  const int64_t m = n_out[0];
  if (levels == 1 && (rows < 1024 || nc[0] > fdwt_chain_max_length(taps, dtype) / 2) &&
      m > 4096) {
    const int64_t want = std::max<int64_t>(cdiv(2048, rows), cdiv(m, 16384));
    int64_t per = std::max<int64_t>(1024, cdiv(m, want));
    per = (per + 1023) & ~(int64_t)1023;
    a.split = (int)per;
    wg = (int)cdiv(m, per);
  }
  if (!a.split) return synthesis_rows(a, rows, dtype, static_cast<hipStream_t>(stream));
  // split mode (one level, long rows): no queued high bands
  a.qslots = 0;
  a.qlevels = 0;
  int capA, capB, capE, capD;
  schain_caps(nc, n_out, levels, taps, off, mode, a.split, &capA, &capB, &capE, &capD);
  a.capA = capA;
  a.capB = capB;
  a.capE = capE;
  a.capD = capD;
  const int cs = compute_size(dtype);
  // A, B, E, ET (ints), F, D, taps
  const size_t lds = (size_t)LREC_BYTES +
                     (size_t)(capA + capB + capE + (2 * capE + 8) + capD + 2 * taps + 4) * cs +
                     (size_t)capE * 4;
  if (!fits_lds((int64_t)lds)) return FDWT_ERR_TOO_LONG;
  // at most 2^32 - 1 threads per launch: consecutive launches over row ranges
  const int64_t per = std::max<int64_t>(1, (int64_t)(0xffffffffu / (unsigned)NT) / wg);
  const int es = dtype_size(dtype);
  for (int64_t r0 = 0; r0 < rows; r0 += per) {
    SChainArgs c = a;
    if (a.approx) c.approx = static_cast<const char*>(a.approx) + r0 * nc[0] * es;
    for (int l = 0; l < levels; ++l)
      if (a.details[l]) c.details[l] = static_cast<const char*>(a.details[l]) + r0 * nc[l] * es;
    c.out = static_cast<char*>(a.out) + r0 * n_out[levels - 1] * es;
    const int rc = dispatch_schain(c, std::min(per, rows - r0), wg, lds, dtype,
                                   static_cast<hipStream_t>(stream));
    if (rc) return rc;
  }
  return 0;
}

extern "C" int fdwt_dwt_analysis(const void* x, void* y0, void* y1, const void* h0,
                                 const void* h1, int64_t rows, int64_t n, int64_t n_out,
                                 int32_t taps, int32_t mode, int32_t off, int32_t dtype,
                                 void* stream) {
  void* det[1] = {y1};
  return fdwt_analysis_chain(x, det, y0, h0, h1, rows, &n, &n_out, 1, taps, mode, off, dtype,
                             stream);
}

extern "C" int fdwt_dwt_synthesis(const void* a, const void* d, void* y, const void* h0,
                                  const void* h1, int64_t rows, int64_t nc, int64_t n,
                                  int32_t taps, int32_t mode, int32_t off, int32_t dtype,
                                  void* stream) {
  const void* det[1] = {d};
  return fdwt_synthesis_chain(a, det, y, h0, h1, rows, &nc, &n, 1, taps, mode, off, dtype,
                              stream);
}

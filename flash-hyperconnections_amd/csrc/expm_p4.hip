// P == 4 kernel (n = 2, 3, 4): one matrix per lane, 64 matrices per
// wavefront.
//
// Each lane keeps its whole 4 x 4 matrix (16 VGPRs; the Frechet kernel keeps
// the D and U blocks, 32 VGPRs) and every product is 64 plain FP32 FMAs with
// compile-time register indices -- no cross-lane traffic, no transposes.  The
// per-matrix scalar work (norm, squaring count, scaling) is done once per
// matrix rather than once per row.
//
// Measured on gfx950: a wave64 FP32 VALU instruction issues every ~3.3 cycles
// at 2 wavefronts per SIMD and ~2.6 at 4; a 4x4x1 FP32 MFMA does 256 FMAs in
// ~8.6 cycles but never overlaps VALU work, so a matrix-core variant (16
// matrices per wavefront, LDS transposes for left operands) has the same
// pipe-time floor and ran slower; DPP-sourced operands run at half rate.  The
// Frechet kernel is VALU-bound at 2 wavefronts per SIMD (~190 VGPRs); the
// forward kernel runs 4 per SIMD and is bound by memory plus its polynomial.
//
// Loads keep raw storage bytes until the group's turn.  Dense operands (64
// packed matrices form one contiguous block) are read with 1 KB per load
// instruction and routed to their lanes through LDS; other vector-class
// operands load their rows or columns per lane; anything else element-wise.
// Stores go through an LDS staging tile so that they are coalesced as well.
//
// Arithmetic is the reference's, element by element (csrc/MatrixExpSmall.cuh:
// 22-106): product entries accumulate k = 0..3 with fmaf from +0, Frechet U
// blocks sum D.U and U.D separately and add them, combines are the
// contracted chain c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 with its zero
// coefficients skipped.  Results are bit-identical to that evaluation up to
// the sign of zero results.  Nothing a matrix computes depends on the batch
// size or on its position in the batch.
#include "fh_kernels.h"

namespace fh {
namespace {

struct M4 {
  float v[16];  // row-major
};

template <bool Pair>
struct PM {
  M4 d;
  M4 u;
};

// Row i of the structured product (D1.D2, D1.U2 + U1.D2): the D and D.U sums
// run in one k loop, U.D in a second, and the two U sums are added last
// (csrc/MatrixExpSmall.cuh:27-49).
template <bool Pair>
__device__ __forceinline__ void pmul_row(const float* xd, const float* xu, const PM<Pair>& y, float* cd, float* cu) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float d = __builtin_fmaf(xd[0], y.d.v[j], 0.f);
    float u = 0.f;
    if constexpr (Pair) u = __builtin_fmaf(xd[0], y.u.v[j], 0.f);
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      d = __builtin_fmaf(xd[k], y.d.v[4 * k + j], d);
      if constexpr (Pair) u = __builtin_fmaf(xd[k], y.u.v[4 * k + j], u);
    }
    cd[j] = d;
    if constexpr (Pair) {
      float v = __builtin_fmaf(xu[0], y.d.v[j], 0.f);
#pragma unroll
      for (int k = 1; k < 4; ++k) v = __builtin_fmaf(xu[k], y.d.v[4 * k + j], v);
      cu[j] = u + v;
    }
  }
}

template <bool Pair>
__device__ __forceinline__ PM<Pair> pmul(const PM<Pair>& x, const PM<Pair>& y) {
  PM<Pair> c;
#pragma unroll
  for (int i = 0; i < 4; ++i) pmul_row<Pair>(&x.d.v[4 * i], &x.u.v[4 * i], y, &c.d.v[4 * i], &c.u.v[4 * i]);
  return c;
}

// Element (i, j) of B(K+1) = c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6, the
// contracted chain of csrc/MatrixExpSmall.cuh:74-77 with zero coefficients
// skipped; c0*I[i][j] is folded at compile time.
template <int K>
__device__ __forceinline__ float comb_d(int e, float a, float a2, float a3, float a6) {
  constexpr float c0 = kCoef[K][0], c1 = kCoef[K][1], c2 = kCoef[K][2], c3 = kCoef[K][3], c6 = kCoef[K][4];
  const bool diag = (e / 4) == (e % 4);
  float t;
  if constexpr (c1 != 0.f) {
    t = __builtin_fmaf(c1, a, c0 * (diag ? 1.f : 0.f));
  } else {
    t = c0 * (diag ? 1.f : 0.f);
  }
  t = __builtin_fmaf(c2, a2, t);
  t = __builtin_fmaf(c3, a3, t);
  if constexpr (c6 != 0.f) t = __builtin_fmaf(c6, a6, t);
  return t;
}
// U blocks have no identity term; their chain starts from c1*A.
template <int K>
__device__ __forceinline__ float comb_u(float a, float a2, float a3, float a6) {
  constexpr float c1 = kCoef[K][1], c2 = kCoef[K][2], c3 = kCoef[K][3], c6 = kCoef[K][4];
  float t;
  if constexpr (c1 != 0.f) {
    t = c1 * a;
    t = __builtin_fmaf(c2, a2, t);
  } else {
    t = c2 * a2;
  }
  t = __builtin_fmaf(c3, a3, t);
  if constexpr (c6 != 0.f) t = __builtin_fmaf(c6, a6, t);
  return t;
}

// Row i of B(K+1) into (bd, bu).
template <int K, bool Pair>
__device__ __forceinline__ void comb_row(const PM<Pair>& a, const PM<Pair>& a2, const PM<Pair>& a3, const PM<Pair>& a6,
                                         int i, float* bd, float* bu) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * i + j;
    bd[j] = comb_d<K>(e, a.d.v[e], a2.d.v[e], a3.d.v[e], a6.d.v[e]);
    if constexpr (Pair) bu[j] = comb_u<K>(a.u.v[e], a2.u.v[e], a3.u.v[e], a6.u.v[e]);
  }
}

template <int K, bool Pair>
__device__ __forceinline__ PM<Pair> comb(const PM<Pair>& a, const PM<Pair>& a2, const PM<Pair>& a3,
                                         const PM<Pair>& a6) {
  PM<Pair> b;
#pragma unroll
  for (int i = 0; i < 4; ++i) comb_row<K, Pair>(a, a2, a3, a6, i, &b.d.v[4 * i], &b.u.v[4 * i]);
  return b;
}

// ---- loads / stores ---------------------------------------------------------
//
// Layout classes (compile time, set by the host for n == 4): kVecRows -- each
// row is one aligned 4-element vector (sc == 1); kVecCols -- each column is
// (sr == 1); kVecNone -- element loads through the strides, n <= 4, padded.

template <typename T>
__device__ __forceinline__ void load_vec4(const typename T::storage* p, float* dst, int stride) {
  using S = typename T::storage;
  typedef S S4 __attribute__((ext_vector_type(4)));
  const S4 w = *reinterpret_cast<const S4*>(p);
  dst[0] = to_f32<T>(w[0]);
  dst[stride] = to_f32<T>(w[1]);
  dst[2 * stride] = to_f32<T>(w[2]);
  dst[3 * stride] = to_f32<T>(w[3]);
}

// Matrix b as row-major FP32 (without the view's sign), zero padded.
template <typename T, int L>
__device__ __forceinline__ M4 load_matrix(const Operand& op, int64_t b, int n, bool valid) {
  using S = typename T::storage;
  M4 m;
#pragma unroll
  for (int e = 0; e < 16; ++e) m.v[e] = 0.f;
  if (!valid) return m;
  const S* base = static_cast<const S*>(op.data) + b * op.sb;
  if constexpr (L == kVecRows) {
#pragma unroll
    for (int i = 0; i < 4; ++i) load_vec4<T>(base + i * op.sr, &m.v[4 * i], 1);
  } else if constexpr (L == kVecCols) {
#pragma unroll
    for (int j = 0; j < 4; ++j) load_vec4<T>(base + j * op.sc, &m.v[j], 4);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i < n && j < n) m.v[4 * i + j] = to_f32<T>(base[i * op.sr + j * op.sc]);
  }
  return m;
}

// Raw storage bytes of one lane's matrix for the vector classes, in the
// memory order of the class (row-major for kVecRows, column-major for
// kVecCols); they are converted only when the group's turn comes, so a
// prefetch never waits for its data.
template <typename T>
struct RawMat {
  static constexpr int kWords = 4 * static_cast<int>(sizeof(typename T::storage));  // 16 or 8
  uint32_t w[kWords];
};

// The four row (column) vectors of matrix b.
template <typename T, int L>
__device__ __forceinline__ RawMat<T> load_lane_raw(const Operand& op, int64_t b, bool valid) {
  using S = typename T::storage;
  RawMat<T> r;
#pragma unroll
  for (int k = 0; k < RawMat<T>::kWords; ++k) r.w[k] = 0u;
  if (!valid) return r;
  const S* base = static_cast<const S*>(op.data) + b * op.sb;
  const int64_t step = L == kVecRows ? op.sr : op.sc;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if constexpr (sizeof(S) == 4) {
      const uint4 x = *reinterpret_cast<const uint4*>(base + v * step);
      r.w[4 * v] = x.x;
      r.w[4 * v + 1] = x.y;
      r.w[4 * v + 2] = x.z;
      r.w[4 * v + 3] = x.w;
    } else {
      const uint2 x = *reinterpret_cast<const uint2*>(base + v * step);
      r.w[2 * v] = x.x;
      r.w[2 * v + 1] = x.y;
    }
  }
  return r;
}

// A full group of a dense operand: this lane's share of the group's
// contiguous block, 16-byte chunks lane, lane + 64, ... -- each load
// instruction reads 1 KB of consecutive memory.
template <typename T>
__device__ __forceinline__ RawMat<T> load_dense_raw(const Operand& op, int64_t group, int lane) {
  using S = typename T::storage;
  constexpr int C = RawMat<T>::kWords / 4;
  const uint4* base = reinterpret_cast<const uint4*>(static_cast<const S*>(op.data) + group * 64 * 16);
  RawMat<T> r;
#pragma unroll
  for (int q = 0; q < C; ++q) {
    const uint4 x = base[q * 64 + lane];
    r.w[4 * q] = x.x;
    r.w[4 * q + 1] = x.y;
    r.w[4 * q + 2] = x.z;
    r.w[4 * q + 3] = x.w;
  }
  return r;
}

// Compiler ordering of the wavefront's LDS accesses (the hardware performs
// one wavefront's LDS operations in issue order).
__device__ __forceinline__ void lds_order() {
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_sched_barrier(0);
}

// Routes a dense group's chunks through the wavefront's LDS tile so that each
// lane ends up with its own matrix: chunk c of matrix m goes to byte
// c * 1040 + 16 * m (rows of 64 chunks padded by 16 bytes, so that both the
// scattered writes and the per-lane reads are free of bank conflicts).
constexpr int kDenseRowBytes = 1024 + 16;

template <typename T>
__device__ __forceinline__ void dense_to_lane(RawMat<T>& r, float* tile, int lane) {
  constexpr int C = RawMat<T>::kWords / 4;
  char* t = reinterpret_cast<char*>(tile);
#pragma unroll
  for (int q = 0; q < C; ++q) {
    const int g = q * 64 + lane;
    *reinterpret_cast<uint4*>(t + (g % C) * kDenseRowBytes + 16 * (g / C)) =
        make_uint4(r.w[4 * q], r.w[4 * q + 1], r.w[4 * q + 2], r.w[4 * q + 3]);
  }
  lds_order();
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const uint4 x = *reinterpret_cast<const uint4*>(t + c * kDenseRowBytes + 16 * lane);
    r.w[4 * c] = x.x;
    r.w[4 * c + 1] = x.y;
    r.w[4 * c + 2] = x.z;
    r.w[4 * c + 3] = x.w;
  }
  lds_order();
}

// Row-major FP32 matrix (without the view's sign) from the raw bytes.
template <typename T, int L>
__device__ __forceinline__ M4 decode(const RawMat<T>& r) {
  using S = typename T::storage;
  M4 m;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float v;
    if constexpr (sizeof(S) == 4) {
      v = __uint_as_float(r.w[e]);
    } else {
      const uint16_t h = static_cast<uint16_t>(r.w[e >> 1] >> (16 * (e & 1)));
      v = to_f32<T>(__builtin_bit_cast(S, h));
    }
    // Memory order: rows class e = 4 * row + col, columns class e = 4 * col + row.
    m.v[L == kVecRows ? e : 4 * (e & 3) + (e >> 2)] = v;
  }
  return m;
}

template <typename T, bool Full>
__device__ __forceinline__ void store_matrix(void* out, int64_t b, int n, const M4& m) {
  using S = typename T::storage;
  if constexpr (Full) {
    typedef S S4 __attribute__((ext_vector_type(4)));
    S* p = static_cast<S*>(out) + b * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      S4 w;
      w[0] = from_f32<T>(m.v[4 * i]);
      w[1] = from_f32<T>(m.v[4 * i + 1]);
      w[2] = from_f32<T>(m.v[4 * i + 2]);
      w[3] = from_f32<T>(m.v[4 * i + 3]);
      *reinterpret_cast<S4*>(p + 4 * i) = w;
    }
  } else {
    S* p = static_cast<S*>(out) + b * n * n;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i < n && j < n) p[i * n + j] = from_f32<T>(m.v[4 * i + j]);
  }
}

constexpr int kP4Waves = 4;  // wavefronts per workgroup
constexpr int kStageStride = 17;  // floats per matrix in the LDS staging tile (odd: conflict-free)

// Per-wavefront LDS tile: the store staging area and, in turn, one (forward)
// or two (Frechet: X and G) dense-group routing areas of 4 x 1040 bytes.
template <bool Pair>
constexpr int kTileFloats = (Pair ? 2 : 1) * kDenseRowBytes > 64 * kStageStride ? (Pair ? 2 : 1) * kDenseRowBytes
                                                                                : 64 * kStageStride;

// Stores the 64 matrices of a full group (n == 4, all rows valid) through
// the wavefront's LDS tile so that the global stores are coalesced: lane l
// writes its matrix with element-wise LDS stores (stride 17, no bank
// conflicts), then each of four passes writes 16 consecutive bytes per lane
// of the group's contiguous output block.
template <typename T>
__device__ __forceinline__ void store_group_staged(void* out, int64_t first, int lane, const M4& m, float* tile) {
  using S = typename T::storage;
  typedef S S4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int e = 0; e < 16; ++e) tile[lane * kStageStride + e] = m.v[e];
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  S* base = static_cast<S*>(out) + first * 16;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int f = pass * 256 + 4 * lane;  // first element of this lane's 4 in the group block
    const int mat = f >> 4;
    const int e = f & 15;
    S4 w;
    w[0] = from_f32<T>(tile[mat * kStageStride + e]);
    w[1] = from_f32<T>(tile[mat * kStageStride + e + 1]);
    w[2] = from_f32<T>(tile[mat * kStageStride + e + 2]);
    w[3] = from_f32<T>(tile[mat * kStageStride + e + 3]);
    *reinterpret_cast<S4*>(base + f) = w;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

// Squaring count of this lane's matrix, or -1 for a non-finite one.  An FP32
// estimate of the column-sum norm decides s whenever it lies clear of a
// squaring boundary (squarings_from_estimate); otherwise the lane takes the
// reference's FP64 norm: column sums over rows as ((x0 + x2) + (x1 + x3))
// with x_r = |A[r][j]| (+ |G[r][j]|) (csrc/MatrixExpSmall.cuh:144-152), whose
// total is finite exactly when every entry is (the non-finite rule of
// :126-140).
template <bool Pair>
__device__ __forceinline__ int lane_squarings(const PM<Pair>& a) {
  uint32_t top = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float c = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      c += __builtin_fabsf(a.d.v[4 * r + j]);
      if constexpr (Pair) c += __builtin_fabsf(a.u.v[4 * r + j]);
    }
    // Bit patterns order non-negative floats, with inf and NaN above all.
    top = max(top, __float_as_uint(c) & 0x7FFFFFFFu);
  }
  int s;
  if (squarings_from_estimate(__uint_as_float(top), s)) return s;
  double norm = 0.;
  double total = 0.;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    double x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = fabs(static_cast<double>(a.d.v[4 * r + j]));
      if constexpr (Pair) x[r] += fabs(static_cast<double>(a.u.v[4 * r + j]));
    }
    const double c = (x[0] + x[2]) + (x[1] + x[3]);
    norm = fmax(norm, c);
    total += c;
  }
  if (!__builtin_isfinite(total)) return -1;
  return squarings_from_norm(norm);
}

// Makes the values of m exist at this point of the program, so that their
// computation is not sunk past later code.
template <bool Pair>
__device__ __forceinline__ void pin(PM<Pair>& m) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    asm volatile("" : "+v"(m.d.v[e]));
    if constexpr (Pair) asm volatile("" : "+v"(m.u.v[e]));
  }
}

// Degree-18 polynomial of this lane's scaled matrix (csrc/MatrixExpSmall.cuh:
// 83-106): A2 = A.A, A3 = A2.A, A6 = A3.A3, A9 = B1.B5 + B4,
// T = B2 + (B3 + A9).A9.  Rows of B1..B4 are formed where they are used, and
// one pass over the rows finishes A9, B3 + A9 and B2 together, so that the
// powers die row by row and only B5 and the three row outputs are kept whole.
template <bool Pair>
__device__ __forceinline__ PM<Pair> t18(const PM<Pair>& a) {
  const PM<Pair> a2 = pmul<Pair>(a, a);
  const PM<Pair> a3 = pmul<Pair>(a2, a);
  const PM<Pair> a6 = pmul<Pair>(a3, a3);
  const PM<Pair> b5 = comb<4, Pair>(a, a2, a3, a6);
  PM<Pair> a9, lhs, b2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float b1d[4], b1u[4], b4d[4], b4u[4];
    comb_row<0, Pair>(a, a2, a3, a6, i, b1d, b1u);
    pmul_row<Pair>(b1d, b1u, b5, &a9.d.v[4 * i], &a9.u.v[4 * i]);
    comb_row<3, Pair>(a, a2, a3, a6, i, b4d, b4u);
    comb_row<2, Pair>(a, a2, a3, a6, i, &lhs.d.v[4 * i], &lhs.u.v[4 * i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * i + j;
      a9.d.v[e] += b4d[j];
      lhs.d.v[e] += a9.d.v[e];
      if constexpr (Pair) {
        a9.u.v[e] += b4u[j];
        lhs.u.v[e] += a9.u.v[e];
      }
    }
    comb_row<1, Pair>(a, a2, a3, a6, i, &b2.d.v[4 * i], &b2.u.v[4 * i]);
  }
  PM<Pair> res;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float qd[4], qu[4];
    pmul_row<Pair>(&lhs.d.v[4 * i], &lhs.u.v[4 * i], a9, qd, qu);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      res.d.v[4 * i + j] = b2.d.v[4 * i + j] + qd[j];
      if constexpr (Pair) res.u.v[4 * i + j] = b2.u.v[4 * i + j] + qu[j];
    }
  }
  return res;
}

// One group's operands between their loads and their turn: raw bytes for the
// vector classes (dense groups still in the loaded chunk order), converted
// matrices for element-wise loads.
template <typename T, bool Pair, int XL, int GL>
struct Staged {
  static constexpr bool kRaw = XL != kVecNone;
  RawMat<T> x, g;
  PM<Pair> m;
  bool dense_x, dense_g;
};

template <typename T, bool Pair, int XL, int GL>
__device__ __forceinline__ void load_group(Staged<T, Pair, XL, GL>& st, const ExpmArgs& args, int64_t group, int lane,
                                           int n) {
  const int64_t b = group * 64 + lane;
  const bool valid = b < args.batch;
  if constexpr (Staged<T, Pair, XL, GL>::kRaw) {
    const bool full = (group + 1) * 64 <= args.batch;
    st.dense_x = full && args.x.dense;
    st.x = st.dense_x ? load_dense_raw<T>(args.x, group, lane) : load_lane_raw<T, XL>(args.x, b, valid);
    if constexpr (Pair) {
      st.dense_g = full && args.g.dense;
      st.g = st.dense_g ? load_dense_raw<T>(args.g, group, lane) : load_lane_raw<T, GL>(args.g, b, valid);
    }
  } else {
    st.m.d = load_matrix<T, XL>(args.x, b, n, valid);
    if constexpr (Pair) st.m.u = load_matrix<T, GL>(args.g, b, n, valid);
  }
}

template <typename T, bool Pair, int XL, int GL>
__device__ __forceinline__ PM<Pair> unstage(Staged<T, Pair, XL, GL>& st, float* tile, int lane) {
  if constexpr (Staged<T, Pair, XL, GL>::kRaw) {
    if (st.dense_x) dense_to_lane<T>(st.x, tile, lane);
    PM<Pair> m;
    m.d = decode<T, XL>(st.x);
    if constexpr (Pair) {
      if (st.dense_g) dense_to_lane<T>(st.g, tile + kDenseRowBytes, lane);
      m.u = decode<T, GL>(st.g);
    }
    return m;
  } else {
    return st.m;
  }
}

// Persistent kernel: each wavefront walks 64-matrix groups with a grid
// stride and keeps the next group's loads in flight while it computes.
template <typename T, bool Pair, int XL, int GL>
__global__ __launch_bounds__(64 * kP4Waves) __attribute__((amdgpu_waves_per_eu(Pair ? 2 : 4, 8))) void expm_p4_kernel(
    ExpmArgs args) {
  __shared__ float tile[kP4Waves][kTileFloats<Pair>];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = (XL != kVecNone) ? 4 : args.n;
  const int64_t groups = (args.batch + 63) / 64;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kP4Waves;
  int64_t group = static_cast<int64_t>(blockIdx.x) * kP4Waves + wave;

  Staged<T, Pair, XL, GL> next;
  if (group < groups) load_group<T, Pair, XL, GL>(next, args, group, lane, n);
  for (; group < groups; group += stride) {
    const int64_t b = group * 64 + lane;
    const bool valid = b < args.batch;
    PM<Pair> cur = unstage<T, Pair, XL, GL>(next, tile[wave], lane);
    const int s = lane_squarings<Pair>(cur);
    const bool bad = s < 0;

    // Scale by 2^-s (csrc/MatrixExpSmall.cuh:157-162) with the views' lazy
    // negation folded into the same exact multiply.
    const float scale = __builtin_ldexpf(1.f, bad ? 0 : -s);
    const float scale_x = scale * args.x.sign;
    const float scale_g = scale * args.g.sign;
    PM<Pair> a;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      a.d.v[e] = cur.d.v[e] * scale_x;
      if constexpr (Pair) a.u.v[e] = cur.u.v[e] * scale_g;
    }

    // Next group's loads: before the polynomial in the forward kernel, which
    // has registers to spare; after it in the Frechet kernel, where the
    // polynomial sets the register peak.  The staged bytes must not stay live
    // past this point, so the last group clears them instead of keeping them.
    auto prefetch = [&]() {
      if (group + stride < groups) {
        load_group<T, Pair, XL, GL>(next, args, group + stride, lane, n);
      } else {
        next = Staged<T, Pair, XL, GL>{};
      }
    };
    if constexpr (!Pair) prefetch();
    PM<Pair> res = t18<Pair>(a);
    pin<Pair>(res);
    if constexpr (Pair) prefetch();

    // s squarings per matrix (csrc/MatrixExpSmall.cuh:168); the wavefront
    // loops while any of its matrices still needs one, the others masked off.
    for (int it = 0; __builtin_amdgcn_ballot_w64(it < s) != 0; ++it) {
      if (it < s) res = pmul<Pair>(res, res);
    }

    M4 outm = Pair ? res.u : res.d;
    if (bad) {
#pragma unroll
      for (int e = 0; e < 16; ++e) outm.v[e] = __builtin_nanf("");
    }
    if constexpr (XL != kVecNone) {
      if ((group + 1) * 64 <= args.batch) {
        store_group_staged<T>(args.out, b - lane, lane, outm, tile[wave]);
      } else if (valid) {
        store_matrix<T, true>(args.out, b, n, outm);
      }
    } else {
      if (valid) store_matrix<T, false>(args.out, b, n, outm);
    }
    if (valid && args.s_out) args.s_out[b] = s;
  }
}

template <typename T, bool Pair, int XL, int GL>
hipError_t launch_p4_l(const ExpmArgs& args, hipStream_t stream) {
  // Persistent grid: as many workgroups as the device keeps resident at once.
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_p4_kernel<T, Pair, XL, GL>), 64 * kP4Waves);
  const int64_t groups = (args.batch + 63) / 64;
  int64_t grid = (groups + kP4Waves - 1) / kP4Waves;
  if (grid > resident) grid = resident;
  hipLaunchKernelGGL((expm_p4_kernel<T, Pair, XL, GL>), dim3(static_cast<unsigned>(grid)), dim3(64 * kP4Waves), 0,
                     stream, args);
  return hipGetLastError();
}

// n < 4 or an unclassified stride pattern takes the element-wise loader; for
// n == 4 each operand is classified independently (the output is row-major).
template <typename T, bool Pair>
hipError_t launch_p4_t(const ExpmArgs& args, hipStream_t stream) {
  const int xl = args.n == 4 ? args.x.vec : kVecNone;
  const int gl = (Pair && args.n == 4) ? args.g.vec : kVecNone;
  if (xl == kVecNone || (Pair && gl == kVecNone)) return launch_p4_l<T, Pair, kVecNone, kVecNone>(args, stream);
  if constexpr (Pair) {
    if (xl == kVecRows) {
      return gl == kVecRows ? launch_p4_l<T, Pair, kVecRows, kVecRows>(args, stream)
                            : launch_p4_l<T, Pair, kVecRows, kVecCols>(args, stream);
    }
    return gl == kVecRows ? launch_p4_l<T, Pair, kVecCols, kVecRows>(args, stream)
                          : launch_p4_l<T, Pair, kVecCols, kVecCols>(args, stream);
  } else {
    return xl == kVecRows ? launch_p4_l<T, Pair, kVecRows, kVecNone>(args, stream)
                          : launch_p4_l<T, Pair, kVecCols, kVecNone>(args, stream);
  }
}

}  // namespace

hipError_t launch_p4(const ExpmArgs& args, int dtype, bool pair, hipStream_t stream) {
  if (dtype == F32::code) return pair ? launch_p4_t<F32, true>(args, stream) : launch_p4_t<F32, false>(args, stream);
  if (dtype == BF16::code) return pair ? launch_p4_t<BF16, true>(args, stream) : launch_p4_t<BF16, false>(args, stream);
  return pair ? launch_p4_t<F16, true>(args, stream) : launch_p4_t<F16, false>(args, stream);
}

}  // namespace fh

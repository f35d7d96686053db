// P == 4 kernel (n = 2, 3, 4): one matrix per lane, 64 matrices per
// wavefront.
//
// Each lane keeps its whole 4 x 4 matrix (16 VGPRs; the Frechet kernel keeps
// the D and U blocks, 32 VGPRs) and every product is 64 plain FP32 FMAs with
// compile-time register indices -- no cross-lane traffic, no transposes.  The
// per-matrix scalar work (norm, squaring count, scaling) is done once per
// matrix rather than once per row.
//
// What bounds it on gfx950 (measured): a wave64 FP32 VALU instruction issues
// every ~4.1 cycles per SIMD whatever the occupancy (16 lanes per clock,
// unpacked), FP32 MFMA does not overlap VALU work on the same SIMD, and a
// VALU instruction with 16 or fewer active lanes costs ~5x a full one.  So the
// kernel is shaped to issue as few VALU instructions as possible, all with
// full exec masks:
//  * operand classes (row / column vectors, dense 64-matrix blocks) are
//    template parameters, so no register shuffles join alternative load paths;
//  * loads and stores go through buffer resources with the group offset in an
//    SGPR: no VALU address arithmetic;
//  * raw storage bytes are staged as 16-byte tuples until the group's turn, so
//    a prefetch stays in flight across the previous group's polynomial and
//    feeds LDS writes without repacking;
//  * squarings run over the full wavefront on ping-pong register sets; each
//    lane keeps (by a select) the result of its own last squaring, and the
//    wavefront's last squaring forms only the block the output needs.
// The one partial group of a batch (B % 64 matrices) takes a separate, cold
// path with per-element loads and stores.
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

typedef uint32_t U32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t U32x2 __attribute__((ext_vector_type(2)));

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
// (csrc/MatrixExpSmall.cuh:27-49).  WantD = false skips the D block (a last
// squaring whose D block nothing reads).
template <bool Pair, bool WantD = true>
__device__ __forceinline__ void pmul_row(const float* xd, const float* xu, const PM<Pair>& y, float* cd, float* cu) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (WantD) {
      float d = __builtin_fmaf(xd[0], y.d.v[j], 0.f);
#pragma unroll
      for (int k = 1; k < 4; ++k) d = __builtin_fmaf(xd[k], y.d.v[4 * k + j], d);
      cd[j] = d;
    }
    if constexpr (Pair) {
      float u = __builtin_fmaf(xd[0], y.u.v[j], 0.f);
#pragma unroll
      for (int k = 1; k < 4; ++k) u = __builtin_fmaf(xd[k], y.u.v[4 * k + j], u);
      float v = __builtin_fmaf(xu[0], y.d.v[j], 0.f);
#pragma unroll
      for (int k = 1; k < 4; ++k) v = __builtin_fmaf(xu[k], y.d.v[4 * k + j], v);
      cu[j] = u + v;
    }
  }
}

template <bool Pair, bool WantD = true>
__device__ __forceinline__ PM<Pair> pmul(const PM<Pair>& x, const PM<Pair>& y) {
  PM<Pair> c;
#pragma unroll
  for (int i = 0; i < 4; ++i) pmul_row<Pair, WantD>(&x.d.v[4 * i], &x.u.v[4 * i], y, &c.d.v[4 * i], &c.u.v[4 * i]);
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
    float c = __builtin_fabsf(a.d.v[j]) + __builtin_fabsf(a.d.v[4 + j]);
    c += __builtin_fabsf(a.d.v[8 + j]);
    c += __builtin_fabsf(a.d.v[12 + j]);
    if constexpr (Pair) {
#pragma unroll
      for (int r = 0; r < 4; ++r) c += __builtin_fabsf(a.u.v[4 * r + j]);
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

// ---- operand staging --------------------------------------------------------
//
// Layout classes (compile time, set by the host for n == 4): kVecRows -- each
// row is one aligned 4-element vector (sc == 1); kVecCols -- each column is
// (sr == 1); kVecNone -- element loads through the strides, n <= 4, padded.
// Dense (compile time as well): the 64 matrices of a group are one contiguous
// block of 64 * 16 elements in the class's memory order.

// Raw storage of one lane's share of a group: C 16-byte tuples, where C is the
// number of tuples one matrix spans (4 in FP32, 2 in FP16/BF16).
template <typename T>
struct Raw {
  static constexpr int C = static_cast<int>(sizeof(typename T::storage));
  uint4 q[C];
};

// Dense group: tuples lane, lane + 64, ... of the group's contiguous block, so
// that each load instruction reads 1 KB of consecutive memory.  `group_bytes`
// is the uniform byte offset of the group in the operand.
template <typename T>
__device__ __forceinline__ Raw<T> load_dense(__amdgpu_buffer_rsrc_t rs, int lane, int32_t group_bytes) {
  Raw<T> r;
#pragma unroll
  for (int c = 0; c < Raw<T>::C; ++c) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * lane, group_bytes + 1024 * c, 0);
    r.q[c] = make_uint4(v[0], v[1], v[2], v[3]);
  }
  return r;
}

// Per-lane vectors: the matrix's four rows (kVecRows) or columns (kVecCols),
// 4 elements each, at byte offset `mat_bytes` (uniform part `group_bytes`).
template <typename T, int L>
__device__ __forceinline__ Raw<T> load_lane(__amdgpu_buffer_rsrc_t rs, int32_t mat_bytes, int32_t step_bytes,
                                            int32_t group_bytes) {
  Raw<T> r;
  if constexpr (sizeof(typename T::storage) == 4) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(rs, mat_bytes + v * step_bytes, group_bytes, 0);
      r.q[v] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const auto x0 = __builtin_amdgcn_raw_buffer_load_b64(rs, mat_bytes + (2 * h) * step_bytes, group_bytes, 0);
      const auto x1 = __builtin_amdgcn_raw_buffer_load_b64(rs, mat_bytes + (2 * h + 1) * step_bytes, group_bytes, 0);
      r.q[h] = make_uint4(x0[0], x0[1], x1[0], x1[1]);
    }
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

// Routes a dense group's tuples through the wavefront's LDS tile so that each
// lane ends up with its own matrix: tuple c of matrix m goes to byte
// c * 1040 + 16 * m (rows of 64 tuples padded by 16 bytes, so that both the
// scattered writes and the per-lane reads are free of bank conflicts).
constexpr int kDenseRowBytes = 1024 + 16;

template <typename T>
__device__ __forceinline__ void dense_to_lane(Raw<T>& r, char* tile, int lane) {
  constexpr int C = Raw<T>::C;
#pragma unroll
  for (int q = 0; q < C; ++q) {
    const int g = q * 64 + lane;  // tuple g of the block: matrix g / C, tuple g % C of it
    *reinterpret_cast<uint4*>(tile + (g % C) * kDenseRowBytes + 16 * (g / C)) = r.q[q];
  }
  lds_order();
#pragma unroll
  for (int c = 0; c < C; ++c) r.q[c] = *reinterpret_cast<const uint4*>(tile + c * kDenseRowBytes + 16 * lane);
  lds_order();
}

// Row-major FP32 matrix (without the view's sign) from one matrix's tuples in
// the class's memory order (rows: e = 4 * row + col; columns: e = 4 * col + row).
template <typename T, int L>
__device__ __forceinline__ M4 decode(const Raw<T>& r) {
  using S = typename T::storage;
  M4 m;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float v;
    if constexpr (sizeof(S) == 4) {
      const uint4& t = r.q[e >> 2];
      const uint32_t w = (e & 3) == 0 ? t.x : (e & 3) == 1 ? t.y : (e & 3) == 2 ? t.z : t.w;
      v = __uint_as_float(w);
    } else {
      const uint4& t = r.q[e >> 3];
      const int k = (e >> 1) & 3;
      const uint32_t w = k == 0 ? t.x : k == 1 ? t.y : k == 2 ? t.z : t.w;
      const uint16_t h = static_cast<uint16_t>(w >> (16 * (e & 1)));
      v = to_f32<T>(__builtin_bit_cast(S, h));
    }
    m.v[L == kVecRows ? e : 4 * (e & 3) + (e >> 2)] = v;
  }
  return m;
}

// Matrix b as row-major FP32 (without the view's sign), zero padded, read
// element by element through the strides (n <= 4; any strides).
template <typename T>
__device__ __forceinline__ M4 load_elements(const Operand& op, int64_t b, int n) {
  using S = typename T::storage;
  M4 m;
#pragma unroll
  for (int e = 0; e < 16; ++e) m.v[e] = 0.f;
  const S* base = static_cast<const S*>(op.data) + b * op.sb;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (i < n && j < n) m.v[4 * i + j] = to_f32<T>(base[i * op.sr + j * op.sc]);
  return m;
}

template <typename T>
__device__ __forceinline__ void store_elements(void* out, int64_t b, int n, const M4& m) {
  using S = typename T::storage;
  S* p = static_cast<S*>(out) + b * n * n;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (i < n && j < n) p[i * n + j] = from_f32<T>(m.v[4 * i + j]);
}

constexpr int kP4Waves = 4;       // wavefronts per workgroup
constexpr int kStageStride = 17;  // floats per matrix in the LDS staging tile (odd: conflict-free)

// Per-wavefront LDS tile: the store staging area and, in turn, one (forward)
// or two (Frechet: X and G) dense-group routing areas of 4 x 1040 bytes.
template <bool Pair>
constexpr int kTileBytes = (Pair ? 2 : 1) * 4 * kDenseRowBytes > 4 * 64 * kStageStride
                               ? (Pair ? 2 : 1) * 4 * kDenseRowBytes
                               : 4 * 64 * kStageStride;

// Stores the 64 matrices of a full group (n == 4) through the wavefront's LDS
// tile so that the global stores are coalesced: lane l has written its matrix
// with element-wise LDS stores (stage_lane: stride 17, no bank conflicts);
// then in each of four passes every lane stores 4 consecutive elements, pass p
// covering elements [256 p, 256 p + 256) of the group's contiguous block.
__device__ __forceinline__ void stage_lane(float* tile, int lane, const M4& m) {
#pragma unroll
  for (int e = 0; e < 16; ++e) tile[lane * kStageStride + e] = m.v[e];
}

template <typename T>
__device__ __forceinline__ void store_group(__amdgpu_buffer_rsrc_t out, int32_t group_bytes, int lane, float* tile) {
  lds_order();
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int f = pass * 256 + 4 * lane;  // first element of this lane's 4 in the group block
    const int mat = f >> 4;
    const int e = f & 15;
    const float v0 = tile[mat * kStageStride + e];
    const float v1 = tile[mat * kStageStride + e + 1];
    const float v2 = tile[mat * kStageStride + e + 2];
    const float v3 = tile[mat * kStageStride + e + 3];
    if constexpr (sizeof(typename T::storage) == 4) {
      const U32x4 w = {__float_as_uint(v0), __float_as_uint(v1), __float_as_uint(v2), __float_as_uint(v3)};
      __builtin_amdgcn_raw_buffer_store_b128(w, out, 4 * f, group_bytes, 0);
    } else {
      const uint32_t lo = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v0))) |
                          (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v1))) << 16);
      const uint32_t hi = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v2))) |
                          (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v3))) << 16);
      const U32x2 w = {lo, hi};
      __builtin_amdgcn_raw_buffer_store_b64(w, out, 2 * f, group_bytes, 0);
    }
  }
  lds_order();
}

// Scale by 2^-s (csrc/MatrixExpSmall.cuh:157-162) with the views' lazy
// negation folded into the same exact multiply; a wavefront whose matrices
// all have s == 0 and no negation skips the multiplies (x * 1 == x).
template <bool Pair>
__device__ __forceinline__ PM<Pair> scaled(const PM<Pair>& cur, int s, float sign_x, float sign_g) {
  const bool bad = s < 0;
  const bool trivial = __builtin_amdgcn_ballot_w64(s > 0) == 0 && sign_x == 1.f && (!Pair || sign_g == 1.f);
  if (trivial) return cur;
  const float scale = __builtin_ldexpf(1.f, bad ? 0 : -s);
  const float sx = scale * sign_x;
  const float sg = scale * sign_g;
  PM<Pair> a;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    a.d.v[e] = cur.d.v[e] * sx;
    if constexpr (Pair) a.u.v[e] = cur.u.v[e] * sg;
  }
  return a;
}

// The output block of exp (D) or of the Frechet derivative (U) after each
// lane's own number of squarings (csrc/MatrixExpSmall.cuh:168; s < 0, a
// non-finite matrix, squares like s = 0), handed to `sink`.  All lanes square in
// every round up to the wavefront's largest s (smax); a lane keeps, by a
// select, the output block of the round that completes its count; the
// wavefront's last round forms only the output block.  The rounds after the
// first go in pairs so that the loop-carried set is rebuilt in place, and every
// exit hands its registers to the sink as they are, with no per-lane branch
// between, so that no path copies the output block to meet another.
__device__ __forceinline__ bool any_lane(bool c) { return __builtin_amdgcn_ballot_w64(c) != 0; }

template <bool Pair>
__device__ __forceinline__ const M4& out_block(const PM<Pair>& m) {
  if constexpr (Pair) {
    return m.u;
  } else {
    return m.d;
  }
}

// x.x, output block only (the forward needs D, the Frechet kernel U = D.U + U.D).
template <bool Pair>
__device__ __forceinline__ M4 square_out(const PM<Pair>& x) {
  return out_block<Pair>(pmul<Pair, !Pair>(x, x));
}

__device__ __forceinline__ void keep_if(M4& out, const M4& m, bool c) {
#pragma unroll
  for (int e = 0; e < 16; ++e) out.v[e] = c ? m.v[e] : out.v[e];
}

__device__ __forceinline__ M4 pick(bool c, const M4& a, const M4& b) {
  M4 r;
#pragma unroll
  for (int e = 0; e < 16; ++e) r.v[e] = c ? a.v[e] : b.v[e];
  return r;
}

template <bool Pair, class Sink>
__device__ __forceinline__ void squarings(const PM<Pair>& t, int s_lane, Sink&& sink) {
  const int s = s_lane < 0 ? 0 : s_lane;
  int smax = 0;
  while (any_lane(s > smax)) ++smax;
  if (smax == 0) {
    sink(out_block<Pair>(t));
    return;
  }
  if (smax == 1) {
    sink(pick(s == 1, square_out<Pair>(t), out_block<Pair>(t)));
    return;
  }
  PM<Pair> x = pmul<Pair>(t, t);  // round 1
  M4 out = pick(s == 1, out_block<Pair>(x), out_block<Pair>(t));
  int k = 1;  // rounds done
  for (; k + 2 < smax; k += 2) {
    const PM<Pair> y = pmul<Pair>(x, x);
    keep_if(out, out_block<Pair>(y), s == k + 1);
    x = pmul<Pair>(y, y);
    keep_if(out, out_block<Pair>(x), s == k + 2);
  }
  if (smax - k == 2) {
    const PM<Pair> y = pmul<Pair>(x, x);
    keep_if(out, out_block<Pair>(y), s == k + 1);
    keep_if(out, square_out<Pair>(y), s == k + 2);
    sink(out);
  } else {
    keep_if(out, square_out<Pair>(x), s == k + 1);
    sink(out);
  }
}

// exp (or the Frechet block) of one lane's unscaled operand, handed to sink;
// returns the lane's squaring count, -1 for a non-finite matrix, whose output
// the caller replaces by NaN (csrc/MatrixExpSmall.cuh:126-140).
template <bool Pair, class Sink>
__device__ __forceinline__ int expm_lane(const PM<Pair>& cur, float sign_x, float sign_g, Sink&& sink) {
  const int s = lane_squarings<Pair>(cur);
  const PM<Pair> a = scaled<Pair>(cur, s, sign_x, sign_g);
  squarings<Pair>(t18<Pair>(a), s, sink);
  return s;
}

// The partial last group (lanes with b < batch) and every group of an
// element-class operand: per-element loads and stores through the strides.
template <typename T, bool Pair>
__device__ __forceinline__ void expm_group_elements(const ExpmArgs& args, int64_t group, int lane) {
  const int64_t b = group * 64 + lane;
  const bool valid = b < args.batch;
  PM<Pair> cur;
  if (valid) {
    cur.d = load_elements<T>(args.x, b, args.n);
    if constexpr (Pair) cur.u = load_elements<T>(args.g, b, args.n);
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      cur.d.v[e] = 0.f;
      if constexpr (Pair) cur.u.v[e] = 0.f;
    }
  }
  M4 res;
  const int s = expm_lane<Pair>(cur, args.x.sign, args.g.sign, [&](const M4& out) { res = out; });
  if (s < 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) res.v[e] = __builtin_nanf("");
  }
  if (valid) {
    store_elements<T>(args.out, b, args.n, res);
    if (args.s_out) args.s_out[b] = s;
  }
}

// Per-operand addressing of the vector classes: a buffer resource over the
// operand, the lane's byte offset within a group and the group's byte stride.
struct VecSrc {
  __amdgpu_buffer_rsrc_t rs;
  int32_t lane_bytes;   // dense: unused; per lane: lane * sb * es
  int32_t step_bytes;   // per lane: bytes between the four vectors (sr or sc)
  int32_t group_bytes;  // bytes between consecutive groups (64 * sb * es)
};

template <typename T>
__device__ __forceinline__ VecSrc make_vec_src(const Operand& op, int L, int lane) {
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  VecSrc v;
  v.rs = make_rsrc(op.data, 0x7FFFFFFFu);
  v.lane_bytes = static_cast<int32_t>(lane * op.sb * es);
  v.step_bytes = static_cast<int32_t>((L == kVecRows ? op.sr : op.sc) * es);
  v.group_bytes = static_cast<int32_t>(64 * op.sb * es);
  return v;
}

template <typename T, int L, bool Dense>
__device__ __forceinline__ Raw<T> load_vec(const VecSrc& src, int lane, int32_t group) {
  const int32_t off = group * src.group_bytes;
  if constexpr (Dense) {
    return load_dense<T>(src.rs, lane, off);
  } else {
    return load_lane<T, L>(src.rs, src.lane_bytes, src.step_bytes, off);
  }
}

// Persistent kernel over the full groups of a vector-class batch (n == 4):
// each wavefront walks 64-matrix groups with a grid stride and keeps the next
// group's loads in flight while it computes.  XD / GD: the operand is dense.
template <typename T, bool Pair, int XL, int GL, bool XD, bool GD>
__global__ __launch_bounds__(64 * kP4Waves) __attribute__((amdgpu_waves_per_eu(Pair ? 2 : 4, 8))) void expm_p4_kernel(
    ExpmArgs args) {
  __shared__ __attribute__((aligned(16))) char tile_mem[kP4Waves][kTileBytes<Pair>];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: offsets stay in SGPRs
  char* tile = tile_mem[wave];
  // Groups fit in 32 bits: the host takes this kernel only for operands below 2 GiB.
  const int32_t full = static_cast<int32_t>(args.batch / 64);
  const int32_t stride = static_cast<int32_t>(gridDim.x) * kP4Waves;
  int32_t group = static_cast<int32_t>(blockIdx.x) * kP4Waves + wave;
  constexpr int es = static_cast<int>(sizeof(typename T::storage));

  const VecSrc sx = make_vec_src<T>(args.x, XL, lane);
  VecSrc sg = sx;
  if constexpr (Pair) sg = make_vec_src<T>(args.g, GL, lane);
  const __amdgpu_buffer_rsrc_t out_rs = make_rsrc(args.out, 0x7FFFFFFFu);

  Raw<T> nx, ng;
  if (group < full) {
    nx = load_vec<T, XL, XD>(sx, lane, group);
    if constexpr (Pair) ng = load_vec<T, GL, GD>(sg, lane, group);
  }
  for (; group < full; group += stride) {
    Raw<T> rx = nx, rg = ng;
    if constexpr (XD) dense_to_lane<T>(rx, tile, lane);
    if constexpr (Pair && GD) dense_to_lane<T>(rg, tile + 4 * kDenseRowBytes, lane);
    PM<Pair> cur;
    cur.d = decode<T, XL>(rx);
    if constexpr (Pair) cur.u = decode<T, GL>(rg);
    // Next group's loads, in flight across this group's polynomial; the last
    // round reloads the final group instead of branching around the loads.
    const int32_t next = group + stride < full ? group + stride : full - 1;
    nx = load_vec<T, XL, XD>(sx, lane, next);
    if constexpr (Pair) ng = load_vec<T, GL, GD>(sg, lane, next);
    float* stage = reinterpret_cast<float*>(tile);
    const int s = expm_lane<Pair>(cur, args.x.sign, args.g.sign, [&](const M4& out) { stage_lane(stage, lane, out); });
    if (s < 0) {  // rare: overwrite the staged block with NaN
      M4 nan;
#pragma unroll
      for (int e = 0; e < 16; ++e) nan.v[e] = __builtin_nanf("");
      stage_lane(stage, lane, nan);
    }
    store_group<T>(out_rs, group * 64 * 16 * es, lane, stage);
    if (args.s_out) args.s_out[static_cast<int64_t>(group) * 64 + lane] = s;
  }
  // The partial last group, if any, belongs to the wavefront whose walk reaches it.
  if (group == full && static_cast<int64_t>(full) * 64 < args.batch) expm_group_elements<T, Pair>(args, group, lane);
}

// Every group of an element-class batch (n < 4 or strides no vector class
// fits): per-element loads and stores.
template <typename T, bool Pair>
__global__ __launch_bounds__(64 * kP4Waves) __attribute__((amdgpu_waves_per_eu(Pair ? 2 : 4, 8))) void expm_p4_elem_kernel(
    ExpmArgs args) {
  const int lane = threadIdx.x & 63;
  const int64_t groups = (args.batch + 63) / 64;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kP4Waves;
  for (int64_t group = static_cast<int64_t>(blockIdx.x) * kP4Waves + (threadIdx.x >> 6); group < groups;
       group += stride)
    expm_group_elements<T, Pair>(args, group, lane);
}

template <typename K>
hipError_t launch_persistent(K kernel, int64_t groups, const ExpmArgs& args, hipStream_t stream, int64_t resident) {
  int64_t grid = (groups + kP4Waves - 1) / kP4Waves;
  if (grid > resident) grid = resident;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(64 * kP4Waves), 0, stream, args);
  return hipGetLastError();
}

template <typename T, bool Pair, int XL, int GL, bool XD, bool GD>
hipError_t launch_vec(const ExpmArgs& args, hipStream_t stream) {
  // Persistent grid: as many workgroups as the device keeps resident at once.
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_p4_kernel<T, Pair, XL, GL, XD, GD>), 64 * kP4Waves);
  // Full groups, plus the wavefront after them for a partial last group.
  const int64_t groups = args.batch / 64 + (args.batch % 64 != 0);
  return launch_persistent(expm_p4_kernel<T, Pair, XL, GL, XD, GD>, groups, args, stream, resident);
}

template <typename T, bool Pair, int XL, int GL>
hipError_t launch_vec_dense(const ExpmArgs& args, hipStream_t stream) {
  const bool xd = args.x.dense != 0;
  const bool gd = Pair && args.g.dense != 0;
  if (xd) {
    if constexpr (Pair) {
      return gd ? launch_vec<T, Pair, XL, GL, true, true>(args, stream)
                : launch_vec<T, Pair, XL, GL, true, false>(args, stream);
    } else {
      return launch_vec<T, Pair, XL, GL, true, false>(args, stream);
    }
  }
  if constexpr (Pair) {
    if (gd) return launch_vec<T, Pair, XL, GL, false, true>(args, stream);
  }
  return launch_vec<T, Pair, XL, GL, false, false>(args, stream);
}

// The vector classes address an operand through a buffer resource with 32-bit
// offsets: every byte a group touches must lie below 2^31 with non-negative
// strides; otherwise the element kernel (64-bit indexing) runs.
bool vec_addressable(const Operand& op, int64_t batch, int es) {
  if (op.sb < 0 || op.sr < 0 || op.sc < 0) return false;
  const int64_t groups = (batch + 63) / 64;
  const int64_t last = (groups * 64 - 1) * op.sb + 3 * (op.sr + op.sc) + 4;
  return last * es < (int64_t{1} << 31) - 1024;
}

template <typename T, bool Pair>
hipError_t launch_p4_t(const ExpmArgs& args, hipStream_t stream) {
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  int xl = args.n == 4 ? args.x.vec : kVecNone;
  int gl = (Pair && args.n == 4) ? args.g.vec : kVecNone;
  const bool addressable = vec_addressable(args.x, args.batch, es) && (!Pair || vec_addressable(args.g, args.batch, es)) &&
                           args.batch * 16 * es < (int64_t{1} << 31) - 1024;
  if (xl == kVecNone || (Pair && gl == kVecNone) || !addressable) {
    static const int64_t resident =
        resident_blocks(reinterpret_cast<const void*>(&expm_p4_elem_kernel<T, Pair>), 64 * kP4Waves);
    return launch_persistent(expm_p4_elem_kernel<T, Pair>, (args.batch + 63) / 64, args, stream, resident);
  }
  if constexpr (Pair) {
    if (xl == kVecRows) {
      return gl == kVecRows ? launch_vec_dense<T, Pair, kVecRows, kVecRows>(args, stream)
                            : launch_vec_dense<T, Pair, kVecRows, kVecCols>(args, stream);
    }
    return gl == kVecRows ? launch_vec_dense<T, Pair, kVecCols, kVecRows>(args, stream)
                          : launch_vec_dense<T, Pair, kVecCols, kVecCols>(args, stream);
  } else {
    return xl == kVecRows ? launch_vec_dense<T, Pair, kVecRows, kVecNone>(args, stream)
                          : launch_vec_dense<T, Pair, kVecCols, kVecNone>(args, stream);
  }
}

}  // namespace

hipError_t launch_p4(const ExpmArgs& args, int dtype, bool pair, hipStream_t stream) {
  if (dtype == F32::code) return pair ? launch_p4_t<F32, true>(args, stream) : launch_p4_t<F32, false>(args, stream);
  if (dtype == BF16::code) return pair ? launch_p4_t<BF16, true>(args, stream) : launch_p4_t<BF16, false>(args, stream);
  return pair ? launch_p4_t<F16, true>(args, stream) : launch_p4_t<F16, false>(args, stream);
}

}  // namespace fh

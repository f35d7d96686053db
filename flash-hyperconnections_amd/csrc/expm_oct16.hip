// P == 8 forward kernel (n = 5..8) on the matrix cores: 16 matrices per
// 64-lane wavefront, every product on v_mfma_f32_4x4x1_16b_f32.  (The Frechet
// kernel keeps the 4-matrix layout of expm_oct.hip: its (D, U) pair does not
// fit this layout's registers at more than two wavefronts per SIMD, and a
// wavefront of 16 matrices squares to the largest count of 16 rather than 4.)
//
// Layout: lane l serves matrix b = l / 4 and index q = l % 4; MFMA block b of
// every instruction is matrix b.  An 8 x 8 matrix is a 2 x 2 arrangement of
// 4 x 4 blocks (I, J), beta = 2I + J, held in one of two 16-VGPR layouts:
//   C (columns):  c[4 beta + r] = M[4I + r][4J + q]   (column q of each block)
//   R (rows):     r[4 beta + c] = M[4I + q][4J + c]   (row q of each block)
// The 4x4x1 MFMA multiplies 16 independent 4 x 4 blocks per instruction
// (block b's lanes supply A[i][0] from lane 4b+i and B[0][j] from lane 4b+j;
// D[i][j] lands in lane 4b+j, VGPR i), so output block (I, J) of X.Y is
//   sum over K = 0, 1 and k = 0..3 of  X_IK[:, k] (x) Y_KJ[k, :]
// with A = entry 4(2I+K) + k of X in the R layout and B = entry 4(2K+J) + k
// of Y in the C layout -- both the lane's own registers -- and lands in the C
// layout.  Each output block is one accumulation chain k = 0..7 (K = 0 block
// first) from +0, the reference's order (csrc/MatrixExpSmall.cuh:31-33), each
// step one exact FMA; the four blocks' chains are independent and interleave.
// The one data movement per product is the left operand's C -> R transpose
// (every 4 x 4 block among its 4 lanes) through the wavefront's LDS plane:
// four 16-byte writes and sixteen 4-byte reads per lane, conflict-free -- 2.5x
// less LDS traffic per product than the 4-matrix layout, whose forward waits
// on LDS issue.
//
// Arithmetic is the reference's, element by element (csrc/MatrixExpSmall.cuh:
// 22-106): combines are the contracted chain with zero coefficients skipped,
// the FP64 norm uses the P = 8 butterfly per column.  Results are
// bit-identical to that evaluation (and to expm_oct.hip's forward) up to the
// sign of zero results.  Packed n == 8 batches run in pairs of units ordered
// by squaring count (expm_oct16_sort_kernel), with the same results.
#include "fh_kernels.h"

namespace fh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;     // wavefronts per workgroup
constexpr int kUnit = 16;     // matrices per wavefront
constexpr int kPlane = 1024;  // floats of one 16-matrix LDS plane (4 KB)

struct O16 {
  float v[16];
};

// Compiler ordering of the wavefront's LDS accesses (the hardware performs
// one wavefront's LDS operations in issue order).
__device__ __forceinline__ void lds_order() {
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

// ---- C <-> R transposes through the LDS plane --------------------------------
//
// Block beta of the plane holds 64 16-byte chunks; lane (b, q) writes its four
// values of the block as chunk 4b + (q ^ g(b)), g(b) = ((b >> 1) ^ (b >> 3)) & 3,
// and reads element q of the chunks of lanes (b, c), c = 0..3.  Writes cover
// consecutive chunks; for each read the 32 (or 64) lanes of a wavefront half
// (whole) hit distinct banks of a 32- (64-) bank LDS.
struct Flip {
  int wr;     // float offset of this lane's chunk
  int rd[4];  // float offsets of element q of the chunks of lanes (b, c)
};

__device__ __forceinline__ Flip make_flip(int lane) {
  const int b = lane >> 2, q = lane & 3;
  const int g = ((b >> 1) ^ (b >> 3)) & 3;
  Flip f;
  f.wr = 4 * (4 * b + (q ^ g));
#pragma unroll
  for (int c = 0; c < 4; ++c) f.rd[c] = 4 * (4 * b + (c ^ g)) + q;
  return f;
}

__device__ __forceinline__ void plane_write(const O16& m, float* t, const Flip& f) {
#pragma unroll
  for (int beta = 0; beta < 4; ++beta)
    *reinterpret_cast<float4*>(t + 256 * beta + f.wr) =
        make_float4(m.v[4 * beta], m.v[4 * beta + 1], m.v[4 * beta + 2], m.v[4 * beta + 3]);
}

__device__ __forceinline__ O16 plane_read(const float* t, const Flip& f) {
  O16 m;
#pragma unroll
  for (int beta = 0; beta < 4; ++beta)
#pragma unroll
    for (int c = 0; c < 4; ++c) m.v[4 * beta + c] = t[256 * beta + f.rd[c]];
  return m;
}

// The other layout of the same matrix (C -> R or R -> C).
__device__ __forceinline__ O16 flip(const O16& m, float* t, const Flip& f) {
  plane_write(m, t, f);
  lds_order();
  const O16 r = plane_read(t, f);
  lds_order();
  return r;
}

// X.Y in the C layout from X in the R layout and Y in the C layout.
__device__ __forceinline__ O16 mm(const O16& xr, const O16& yc) {
  v4f acc[4];
#pragma unroll
  for (int beta = 0; beta < 4; ++beta) acc[beta] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int K = 0; K < 2; ++K)
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int I = 0; I < 2; ++I)
#pragma unroll
        for (int J = 0; J < 2; ++J)
          acc[2 * I + J] = __builtin_amdgcn_mfma_f32_4x4x1f32(xr.v[4 * (2 * I + K) + k], yc.v[4 * (2 * K + J) + k],
                                                              acc[2 * I + J], 0, 0, 0);
  O16 p;
#pragma unroll
  for (int beta = 0; beta < 4; ++beta)
#pragma unroll
    for (int r = 0; r < 4; ++r) p.v[4 * beta + r] = acc[beta][r];
  return p;
}

// Entry e of B(K+1) = c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 in the C layout,
// the contracted chain of csrc/MatrixExpSmall.cuh:74-77 with zero
// coefficients skipped.  Diagonal entries sit in blocks 0 and 3 at r == q:
// `dq[r]` is 1 there and 0 elsewhere.
template <int K>
__device__ __forceinline__ float comb_entry(int e, const O16& a, const O16& a2, const O16& a3, const O16& a6,
                                            const float (&dq)[4]) {
  constexpr float c0 = kCoef[K][0], c1 = kCoef[K][1], c2 = kCoef[K][2], c3 = kCoef[K][3], c6 = kCoef[K][4];
  const int beta = e >> 2, r = e & 3;
  // c0 * I, with +0 from a VGPR off the diagonal blocks and where c0 is 0 (see vgpr_zero).
  const float i0 = c0 != 0.f && (beta == 0 || beta == 3) ? c0 * dq[r] : vgpr_zero();
  float t;
  if constexpr (c1 != 0.f) {
    t = __builtin_fmaf(c1, a.v[e], i0);
    t = __builtin_fmaf(c2, a2.v[e], t);
  } else {
    t = __builtin_fmaf(c2, a2.v[e], i0);
  }
  t = __builtin_fmaf(c3, a3.v[e], t);
  if constexpr (c6 != 0.f) t = __builtin_fmaf(c6, a6.v[e], t);
  return t;
}

// Degree-18 polynomial of the scaled matrix (csrc/MatrixExpSmall.cuh:83-106):
// A2 = A.A, A3 = A2.A, A6 = A3.A3, A9 = B1.B5 + B4, T = B2 + (B3 + A9).A9.
// `ar` / `ac`: A in the R / C layout.  Result in the C layout.  B1..B5 are
// formed together, entry by entry, so that each entry of the powers dies as
// soon as its five combinations exist.
__device__ __forceinline__ O16 t18(const O16& ar, const O16& ac, const float (&dq)[4], float* t, const Flip& f) {
  const O16 a2 = mm(ar, ac);
  const O16 a3 = mm(flip(a2, t, f), ac);
  const O16 a6 = mm(flip(a3, t, f), a3);
  O16 b1, b2, b3, b4, b5;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    b1.v[e] = comb_entry<0>(e, ac, a2, a3, a6, dq);
    b2.v[e] = comb_entry<1>(e, ac, a2, a3, a6, dq);
    b3.v[e] = comb_entry<2>(e, ac, a2, a3, a6, dq);
    b4.v[e] = comb_entry<3>(e, ac, a2, a3, a6, dq);
    b5.v[e] = comb_entry<4>(e, ac, a2, a3, a6, dq);
  }
  O16 a9 = mm(flip(b1, t, f), b5);
#pragma unroll
  for (int e = 0; e < 16; ++e) a9.v[e] += b4.v[e];
  O16 lhs;
#pragma unroll
  for (int e = 0; e < 16; ++e) lhs.v[e] = b3.v[e] + a9.v[e];
  O16 res = mm(flip(lhs, t, f), a9);
#pragma unroll
  for (int e = 0; e < 16; ++e) res.v[e] = b2.v[e] + res.v[e];
  return res;
}

// ---- norm ----------------------------------------------------------------------

// The matrix's 4 lanes are a DPP quad: xor 1 and xor 2 within it.
__device__ __forceinline__ int quad_xor1(int v) { return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int quad_xor2(int v) { return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ double quad_xor1_d(double v) {
  const int2 w = __builtin_bit_cast(int2, v);
  return __builtin_bit_cast(double, make_int2(quad_xor1(w.x), quad_xor1(w.y)));
}
__device__ __forceinline__ double quad_xor2_d(double v) {
  const int2 w = __builtin_bit_cast(int2, v);
  return __builtin_bit_cast(double, make_int2(quad_xor2(w.x), quad_xor2(w.y)));
}

// Squaring count of the lane's matrix, or -1 for a non-finite one.  The lane
// holds columns q (blocks 0 and 2) and 4 + q (blocks 1 and 3) whole.  The FP32
// estimate of the column-sum norm decides s unless it lies near a squaring
// boundary (squarings_from_estimate); then the matrix takes the reference's
// FP64 norm: per column the butterfly ((x0 + x4) + (x2 + x6)) +
// ((x1 + x5) + (x3 + x7)) with x_r = |A[r][j]| (csrc/MatrixExpSmall.cuh:
// 144-152), whose total is finite exactly when every entry is (:126-140).
__device__ __forceinline__ int matrix_squarings(const O16& ac) {
  uint32_t top = 0;
#pragma unroll
  for (int J = 0; J < 2; ++J) {
    float p = 0.f;
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int r = 0; r < 4; ++r) p += __builtin_fabsf(ac.v[4 * (2 * I + J) + r]);
    // Bit patterns order non-negative floats, with inf and NaN above all.
    top = max(top, __float_as_uint(p) & 0x7FFFFFFFu);
  }
  top = max(top, static_cast<uint32_t>(quad_xor1(static_cast<int>(top))));
  top = max(top, static_cast<uint32_t>(quad_xor2(static_cast<int>(top))));
  int s;
  const bool decided = squarings_from_estimate(__uint_as_float(top), s);
  if (__builtin_amdgcn_ballot_w64(!decided) == 0) return s;
  // Some matrix needs the exact norm: the whole wavefront computes it (the DPP
  // exchanges need every lane) and the decided matrices keep their estimate.
  double norm = 0.;
  double total = 0.;
#pragma unroll
  for (int J = 0; J < 2; ++J) {
    double x[8];
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int r = 0; r < 4; ++r) x[4 * I + r] = fabs(static_cast<double>(ac.v[4 * (2 * I + J) + r]));
    const double c = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
    norm = fmax(norm, c);
    total += c;
  }
  norm = fmax(norm, quad_xor1_d(norm));
  total = total + quad_xor1_d(total);
  norm = fmax(norm, quad_xor2_d(norm));
  total = total + quad_xor2_d(total);
  if (decided) return s;
  if (!__builtin_isfinite(total)) return -1;
  return squarings_from_norm(norm);
}

// The same count from the R layout: the lane holds rows q (blocks 0, 1) and
// 4 + q (blocks 2, 3) of every column, so each column sum is completed across
// the quad.  The FP64 butterfly ((x0 + x4) + (x2 + x6)) + ((x1 + x5) +
// (x3 + x7)) is the lane's x_q + x_{q+4}, plus the xor-2 partner's pair, plus
// the xor-1 partner's half: every lane of the quad forms the reference's sums
// in the reference's association (addition commutes exactly).  The FP32
// estimate's order differs from matrix_squarings' but stays within its error
// bound, so both decide the same s.
__device__ __forceinline__ int rows_squarings(const O16& ar) {
  uint32_t top = 0;
#pragma unroll
  for (int J = 0; J < 2; ++J)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float p = __builtin_fabsf(ar.v[4 * J + c]) + __builtin_fabsf(ar.v[4 * (2 + J) + c]);
      p += __int_as_float(quad_xor1(__float_as_int(p)));
      p += __int_as_float(quad_xor2(__float_as_int(p)));
      top = max(top, __float_as_uint(p) & 0x7FFFFFFFu);
    }
  int s;
  const bool decided = squarings_from_estimate(__uint_as_float(top), s);
  if (__builtin_amdgcn_ballot_w64(!decided) == 0) return s;
  double norm = 0.;
  double total = 0.;
#pragma unroll
  for (int J = 0; J < 2; ++J)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      double a = fabs(static_cast<double>(ar.v[4 * J + c])) + fabs(static_cast<double>(ar.v[4 * (2 + J) + c]));
      a = a + quad_xor2_d(a);
      a = a + quad_xor1_d(a);
      norm = fmax(norm, a);
      total += a;
    }
  if (decided) return s;
  if (!__builtin_isfinite(total)) return -1;
  return squarings_from_norm(norm);
}

// ---- loads / stores -------------------------------------------------------------
//
// Layout classes (set by the host for n == 8): kVecRows -- every row of a
// matrix is made of aligned 4-element vectors (sc == 1), loaded straight into
// the R layout; kVecCols -- every column is (sr == 1), loaded into the C
// layout; kVecNone -- element loads through the strides into the C layout,
// zero padded for n < 8.  Raw storage bits are kept until the unit's turn.

template <typename T>
struct Raw16 {
  typename T::storage v[16];
};

template <typename T, int L>
__device__ __forceinline__ Raw16<T> load_raw(const Operand& op, int64_t m, int q, int n, bool valid) {
  using S = typename T::storage;
  typedef S S4 __attribute__((ext_vector_type(4)));
  Raw16<T> w;
#pragma unroll
  for (int e = 0; e < 16; ++e) w.v[e] = S{};
  if (!valid) return w;
  const S* base = static_cast<const S*>(op.data) + m * op.sb;
#pragma unroll
  for (int beta = 0; beta < 4; ++beta) {
    const int I = beta >> 1, J = beta & 1;
    if constexpr (L == kVecRows) {  // row 4I + q, columns 4J..4J+3
      const S4 x = *reinterpret_cast<const S4*>(base + (4 * I + q) * op.sr + 4 * J);
#pragma unroll
      for (int c = 0; c < 4; ++c) w.v[4 * beta + c] = x[c];
    } else if constexpr (L == kVecCols) {  // column 4J + q, rows 4I..4I+3
      const S4 x = *reinterpret_cast<const S4*>(base + (4 * J + q) * op.sc + 4 * I);
#pragma unroll
      for (int r = 0; r < 4; ++r) w.v[4 * beta + r] = x[r];
    } else {
      const int col = 4 * J + q;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * I + r;
        if (row < n && col < n) w.v[4 * beta + r] = base[row * op.sr + col * op.sc];
      }
    }
  }
  return w;
}

template <typename T>
__device__ __forceinline__ O16 to_o16(const Raw16<T>& w) {
  O16 m;
#pragma unroll
  for (int e = 0; e < 16; ++e) m.v[e] = to_f32<T>(w.v[e]);
  return m;
}

// ---- per-unit pieces ------------------------------------------------------------

// exp of the lanes' matrices from A in both layouts and their counts: scale
// by 2^-s with the view's lazy negation folded into the same exact multiply
// (csrc/MatrixExpSmall.cuh:157-162), the degree-18 polynomial, then s
// squarings per matrix (:168) -- the wavefront loops while any of its
// matrices still needs one and each keeps its own result.  A non-finite
// matrix (s < 0) gives NaN.  Result in the C layout.
__device__ __forceinline__ O16 forward_lanes(O16 ar, O16 ac, int s, float sign, const float (&dq)[4], float* t,
                                             const Flip& f) {
  const bool bad = s < 0;
  const float scale = __builtin_ldexpf(1.f, bad ? 0 : -s) * sign;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    ac.v[e] *= scale;
    ar.v[e] *= scale;
  }
  O16 res = t18(ar, ac, dq, t, f);
  for (int it = 0; __builtin_amdgcn_ballot_w64(it < s) != 0; ++it) {
    const O16 sq = mm(flip(res, t, f), res);
    const bool keep = it < s;
#pragma unroll
    for (int e = 0; e < 16; ++e) res.v[e] = keep ? sq.v[e] : res.v[e];
  }
  if (bad) {
#pragma unroll
    for (int e = 0; e < 16; ++e) res.v[e] = __builtin_nanf("");
  }
  return res;
}

// Matrix m's result (C layout) into the contiguous n == 8 output: rows 4I + q
// from the R layout, 4 consecutive entries per store.  Every lane takes part
// in the transpose; only `valid` lanes store.
template <typename T>
__device__ __forceinline__ void store_rows(const ExpmArgs& args, const O16& res, int64_t m, int q, bool valid,
                                           float* t, const Flip& f) {
  using S = typename T::storage;
  typedef S S4 __attribute__((ext_vector_type(4)));
  const O16 rows = flip(res, t, f);
  if (valid) {
    S* o = static_cast<S*>(args.out) + m * 64;
#pragma unroll
    for (int beta = 0; beta < 4; ++beta) {
      const int I = beta >> 1, J = beta & 1;
      S4 w;
#pragma unroll
      for (int c = 0; c < 4; ++c) w[c] = from_f32<T>(rows.v[4 * beta + c]);
      __builtin_nontemporal_store(w, reinterpret_cast<S4*>(o + (4 * I + q) * 8 + 4 * J));
    }
  }
}

// One n == 8 unit from its loaded values `lx` (R layout for kVecRows, C
// layout for kVecCols): both layouts, count, exp, store.
template <typename T, int XL>
__device__ __forceinline__ void unit_forward(const ExpmArgs& args, const O16& lx, int64_t unit, int slot, int q,
                                             const float (&dq)[4], float* t, const Flip& f) {
  const int64_t m = unit * kUnit + slot;
  const bool valid = m < args.batch;
  O16 ar, ac;
  if constexpr (XL == kVecRows) {
    ar = lx;
    ac = flip(lx, t, f);
  } else {
    ac = lx;
    ar = flip(lx, t, f);
  }
  const int s = matrix_squarings(ac);
  store_rows<T>(args, forward_lanes(ar, ac, s, args.x.sign, dq, t, f), m, q, valid, t, f);
  if (valid && q == 0 && args.s_out) args.s_out[m] = s;
}

// ---- kernel -----------------------------------------------------------------

// Persistent kernel: each wavefront walks 16-matrix units with a grid stride
// and issues the next unit's loads before computing the current one.
template <typename T, int XL>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(3, 8))) void expm_oct16_kernel(
    ExpmArgs args) {
  __shared__ __attribute__((aligned(16))) float lds[kWaves][kPlane];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* t = lds[wave];
  const int slot = lane >> 2;
  const int q = lane & 3;
  const int n = (XL != kVecNone) ? 8 : args.n;
  const Flip f = make_flip(lane);
  float dq[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) dq[r] = r == q ? 1.f : 0.f;
  const int64_t units = (args.batch + kUnit - 1) / kUnit;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWaves;
  int64_t unit = static_cast<int64_t>(blockIdx.x) * kWaves + wave;

  auto load_unit = [&](int64_t u) {
    const int64_t m = u * kUnit + slot;
    return load_raw<T, XL>(args.x, m, q, n, m < args.batch);
  };

  Raw16<T> next;
  if (unit < units) next = load_unit(unit);
  for (; unit < units; unit += stride) {
    const int64_t m = unit * kUnit + slot;
    const bool valid = m < args.batch;
    const O16 lx = to_o16<T>(next);  // R layout for kVecRows, C layout otherwise
    if (unit + stride < units) next = load_unit(unit + stride);

    O16 ar, ac;
    if constexpr (XL == kVecRows) {
      ar = lx;
      ac = flip(lx, t, f);
    } else {
      ac = lx;
      ar = flip(lx, t, f);
    }

    const int s = matrix_squarings(ac);
    const O16 res = forward_lanes(ar, ac, s, args.x.sign, dq, t, f);
    if constexpr (XL != kVecNone) {
      store_rows<T>(args, res, m, q, valid, t, f);
    } else if (valid) {
      // n < 8: element stores, written out here (behind a helper function the
      // allocator spilled 32 bytes per lane for FP32 and FP16).
      using S = typename T::storage;
      S* o = static_cast<S*>(args.out) + m * n * n;
#pragma unroll
      for (int beta = 0; beta < 4; ++beta) {
        const int I = beta >> 1, J = beta & 1;
        const int col = 4 * J + q;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 4 * I + r;
          if (row < n && col < n) __builtin_nontemporal_store(from_f32<T>(res.v[4 * beta + r]), &o[row * n + col]);
        }
      }
    }
    if (valid && q == 0 && args.s_out) args.s_out[m] = s;
  }
}

// ---- dense n == 8 batches: pairs of units in squaring-count order ------------
//
// A wavefront squares up to the largest count among its 16 matrices, and
// counts spread when norms span decades.  For a dense batch (packed row- or
// column-major 8 x 8 matrices) the kernel stages 32 matrices at a time in the
// wavefront's LDS with buffer-to-LDS loads, computes all 32 counts, ranks the
// matrices by (count, position) with a counting sort over ballots, and runs
// two rounds of 16 in rank order: the first round squares only up to the 16th
// smallest count.  Which MFMA block computes a matrix does not change what it
// computes, so the results are the unordered kernel's bit for bit.

template <typename T>
struct PairImage {
  static constexpr int kMatBytes = 64 * static_cast<int>(sizeof(typename T::storage));  // one matrix
  static constexpr int kChunks = kMatBytes / 16;                                        // 16-byte chunks
  static constexpr int kBytes = 2 * kUnit * kMatBytes;                                   // 32 matrices
  static constexpr int kLoads = kBytes / 1024;  // buffer-to-LDS loads per pair (1 KB each)
};

// Chunk c of matrix id lies at chunk (c + rot(id)) mod kChunks of the
// matrix's LDS area: the rotation spreads the four matrices a quarter
// wavefront reads together (in unit order) over different banks.
template <typename T>
__device__ __forceinline__ int chunk_rot(int id) {
  return (id & 1) + (PairImage<T>::kChunks / 2) * ((id >> 1) & 1);
}

// LDS byte offset of elements e0..e0+3 of storage line `line` (a row for
// kVecRows, a column for kVecCols) of matrix id.
template <typename T>
__device__ __forceinline__ int image_offset(int id, int line, int e0) {
  using Img = PairImage<T>;
  const int byte = (8 * line + e0) * static_cast<int>(sizeof(typename T::storage));
  return Img::kMatBytes * id + 16 * (((byte >> 4) + chunk_rot<T>(id)) & (Img::kChunks - 1)) + (byte & 15);
}

// Matrix id's part for this lane, in the layout its storage gives: R for
// kVecRows, C for kVecCols.
template <typename T, int XL>
__device__ __forceinline__ O16 image_read(const char* img, int id, int q) {
  using S = typename T::storage;
  typedef S S4 __attribute__((ext_vector_type(4)));
  O16 m;
#pragma unroll
  for (int beta = 0; beta < 4; ++beta) {
    const int I = beta >> 1, J = beta & 1;
    const int line = 4 * (XL == kVecRows ? I : J) + q;
    const int e0 = 4 * (XL == kVecRows ? J : I);
    const S4 x = *reinterpret_cast<const S4*>(img + image_offset<T>(id, line, e0));
#pragma unroll
    for (int k = 0; k < 4; ++k) m.v[4 * beta + k] = to_f32<T>(x[k]);
  }
  return m;
}

// The pair's 32 matrices from byte `pair_bytes` of the operand into the
// image: load instruction i has lane l fetch the chunk that belongs at LDS
// chunk 64 i + l.  Each instruction covers 1 KB of consecutive matrices.
template <typename T>
__device__ __forceinline__ void load_pair(U32x4 rs, uint32_t img, int32_t pair_bytes, int lane) {
  using Img = PairImage<T>;
#pragma unroll
  for (int i = 0; i < Img::kLoads; ++i) {
    const int at = 64 * i + lane;
    const int id = at / Img::kChunks;
    const int c = ((at % Img::kChunks) - chunk_rot<T>(id)) & (Img::kChunks - 1);
    lds_load16(rs, img + 1024 * i, Img::kMatBytes * id + 16 * c, pair_bytes);
  }
}

// Persistent kernel over the batch's full pairs (matrices 32 p .. 32 p + 31);
// the last partial pair takes the unordered path.
template <typename T, int XL>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(3, 8))) void expm_oct16_sort_kernel(
    ExpmArgs args) {
  static_assert(XL == kVecRows || XL == kVecCols, "dense operands are row- or column-major");
  using Img = PairImage<T>;
  __shared__ __attribute__((aligned(16))) float lds[kWaves][kPlane];
  __shared__ __attribute__((aligned(16))) char image_mem[kWaves][Img::kBytes];
  __shared__ uint8_t order_mem[kWaves][2 * kUnit];  // matrix by rank
  __shared__ int16_t count_mem[kWaves][2 * kUnit];  // squaring count by matrix
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* t = lds[wave];
  const char* img = image_mem[wave];
  uint8_t* order = order_mem[wave];
  int16_t* count = count_mem[wave];
  const int slot = lane >> 2;
  const int q = lane & 3;
  const Flip f = make_flip(lane);
  float dq[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) dq[r] = r == q ? 1.f : 0.f;
  // Pairs fit in 32 bits: the host takes this kernel only for operands below 2 GiB.
  const int32_t pairs = static_cast<int32_t>(args.batch / (2 * kUnit));
  const int32_t stride = static_cast<int32_t>(gridDim.x) * kWaves;
  int32_t p = static_cast<int32_t>(blockIdx.x) * kWaves + wave;
  const U32x4 xs = rsrc_words(args.x.data);
  const uint32_t img_addr = lds_address(img);
  if (p < pairs) load_pair<T>(xs, img_addr, p * Img::kBytes, lane);
  for (; p < pairs; p += stride) {
    wait_vm<0>();
    lds_order();
    // Counts of matrices slot (first unit) and 16 + slot (second unit).
    int sh[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const O16 lx = image_read<T, XL>(img, kUnit * h + slot, q);
      sh[h] = XL == kVecRows ? rows_squarings(lx) : matrix_squarings(lx);
    }
    // Rank by (count, matrix): counting sort, one ballot per count value and
    // unit; a matrix's four lanes all vote, so lane counts are 4 per matrix.
    const int k0 = sh[0] < 0 ? 0 : sh[0];
    const int k1 = sh[1] < 0 ? 0 : sh[1];
    int r0 = 0, r1 = 0, base = 0;
    for (int v = 0; base < 2 * kUnit; ++v) {
      const uint64_t b0 = __builtin_amdgcn_ballot_w64(k0 == v);
      const uint64_t b1 = __builtin_amdgcn_ballot_w64(k1 == v);
      if (k0 == v) r0 = base + (lanes_below(b0) >> 2);
      base += __builtin_popcountll(b0) >> 2;
      if (k1 == v) r1 = base + (lanes_below(b1) >> 2);
      base += __builtin_popcountll(b1) >> 2;
    }
    if (q == 0) {
      order[r0] = static_cast<uint8_t>(slot);
      order[r1] = static_cast<uint8_t>(kUnit + slot);
      count[slot] = static_cast<int16_t>(sh[0]);  // at most ~130 for finite inputs
      count[kUnit + slot] = static_cast<int16_t>(sh[1]);
    }
    lds_order();
#pragma unroll 1
    for (int r = 0; r < 2; ++r) {
      const int id = order[kUnit * r + slot];
      const int s = count[id];
      const O16 lx = image_read<T, XL>(img, id, q);
      if (r == 1 && p + stride < pairs) {
        // The image's last reads complete before the next pair's loads land in it.
        wait_lds();
        load_pair<T>(xs, img_addr, (p + stride) * Img::kBytes, lane);
      }
      O16 ar, ac;
      if constexpr (XL == kVecRows) {
        ar = lx;
        ac = flip(lx, t, f);
      } else {
        ac = lx;
        ar = flip(lx, t, f);
      }
      const int64_t m = static_cast<int64_t>(p) * (2 * kUnit) + id;
      store_rows<T>(args, forward_lanes(ar, ac, s, args.x.sign, dq, t, f), m, q, true, t, f);
      if (q == 0 && args.s_out) args.s_out[m] = s;
    }
  }
  // The last partial pair's units, if any, belong to the wavefront whose walk
  // reaches the end of the full pairs.
  if (p == pairs) {
    for (int64_t unit = 2 * static_cast<int64_t>(pairs); unit * kUnit < args.batch; ++unit) {
      const int64_t m = unit * kUnit + slot;
      unit_forward<T, XL>(args, to_o16<T>(load_raw<T, XL>(args.x, m, q, 8, m < args.batch)), unit, slot, q, dq, t, f);
    }
  }
}

template <typename T, int XL>
hipError_t launch_l(const ExpmArgs& args, hipStream_t stream) {
  // Persistent grid: as many workgroups as the device keeps resident at once.
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_oct16_kernel<T, XL>), 64 * kWaves);
  const int64_t units = (args.batch + kUnit - 1) / kUnit;
  int64_t grid = (units + kWaves - 1) / kWaves;
  if (grid > resident) grid = resident;
  hipLaunchKernelGGL((expm_oct16_kernel<T, XL>), dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), 0, stream,
                     args);
  return hipGetLastError();
}

template <typename T, int XL>
hipError_t launch_sorted(const ExpmArgs& args, hipStream_t stream) {
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_oct16_sort_kernel<T, XL>), 64 * kWaves);
  // Full pairs, plus the wavefront after them for a partial last pair.
  const int64_t pairs = args.batch / (2 * kUnit) + (args.batch % (2 * kUnit) != 0);
  int64_t grid = (pairs + kWaves - 1) / kWaves;
  if (grid > resident) grid = resident;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((expm_oct16_sort_kernel<T, XL>), dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), 0,
                     stream, args);
  return hipGetLastError();
}

// Dense n == 8 operands below 2 GiB take the count-ordered kernel; n < 8 or
// an unclassified stride pattern takes the element-wise loader.
template <typename T>
hipError_t launch_t(const ExpmArgs& args, hipStream_t stream) {
  const int xl = args.n == 8 ? args.x.vec : kVecNone;
  const int64_t bytes = args.batch * PairImage<T>::kMatBytes;
  if (xl != kVecNone && args.x.dense && bytes < (int64_t{1} << 31) - 1024) {
    return xl == kVecRows ? launch_sorted<T, kVecRows>(args, stream) : launch_sorted<T, kVecCols>(args, stream);
  }
  if (xl == kVecRows) return launch_l<T, kVecRows>(args, stream);
  if (xl == kVecCols) return launch_l<T, kVecCols>(args, stream);
  return launch_l<T, kVecNone>(args, stream);
}

}  // namespace

hipError_t launch_oct16(const ExpmArgs& args, int dtype, hipStream_t stream) {
  if (dtype == F32::code) return launch_t<F32>(args, stream);
  if (dtype == BF16::code) return launch_t<BF16>(args, stream);
  return launch_t<F16>(args, stream);
}

}  // namespace fh

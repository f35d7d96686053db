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
// sign of zero results.
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
  const float i0 = (beta == 0 || beta == 3) ? c0 * dq[r] : 0.f;
  float t;
  if constexpr (c1 != 0.f) {
    t = __builtin_fmaf(c1, a.v[e], i0);
  } else {
    t = i0;
  }
  t = __builtin_fmaf(c2, a2.v[e], t);
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

// ---- kernel -----------------------------------------------------------------

// Persistent kernel: each wavefront walks 16-matrix units with a grid stride
// and issues the next unit's loads before computing the current one.
template <typename T, int XL>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(3, 8))) void expm_oct16_kernel(
    ExpmArgs args) {
  using S = typename T::storage;
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
    const bool bad = s < 0;

    // Scale by 2^-s (csrc/MatrixExpSmall.cuh:157-162) with the view's lazy
    // negation folded into the same exact multiply.
    const float scale = __builtin_ldexpf(1.f, bad ? 0 : -s) * args.x.sign;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      ac.v[e] *= scale;
      ar.v[e] *= scale;
    }

    O16 res = t18(ar, ac, dq, t, f);

    // s squarings per matrix (csrc/MatrixExpSmall.cuh:168); the wavefront
    // loops while any of its matrices still needs one and each keeps its own
    // result.
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
    if constexpr (XL != kVecNone) {
      // n == 8: rows 4I + q from the R layout, 4 consecutive entries per store.
      const O16 rows = flip(res, t, f);
      if (valid) {
        typedef S S4 __attribute__((ext_vector_type(4)));
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
    } else if (valid) {
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

// n < 8 or an unclassified stride pattern takes the element-wise loader.
template <typename T>
hipError_t launch_t(const ExpmArgs& args, hipStream_t stream) {
  const int xl = args.n == 8 ? args.x.vec : kVecNone;
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

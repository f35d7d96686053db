// P == 4 kernel (n = 2, 3, 4): 16 matrices per 64-lane wavefront.
//
// Layout ("quad column layout"): lane l serves matrix slot l/4 of the
// wavefront and column j = l%4 of it; a matrix value M occupies four VGPRs,
// v[r] = M[r][j].  v_mfma_f32_4x4x1_16b_f32 multiplies 16 independent 4 x 4
// blocks per instruction: block b's lanes 4b+i supply A[i][0] and lanes 4b+j
// supply B[0][j], and D[i][j] lands in lane 4b+j, VGPR i -- the same layout
// as the operands here.  Hence
//   X.Y    = sum_k mfma(a = (X^T).v[k], b = Y.v[k])   (C-layout of X.Y)
//   (X.Y)^T = sum_k mfma(a = Y.v[k], b = (X^T).v[k])  (C-layout of (X.Y)^T)
// Both accumulate k = 0..3 in the reference's order (csrc/MatrixExpSmall.cuh:
// 31-33), one fused multiply-add per step.  Left operands are therefore kept
// transposed; a transpose inside a quad costs 8 DPP moves and 8 selects.
//
// The polynomial's linear combinations B2..B5 run on the same MFMA: with the
// A operand set to the coefficient column (lane 4b+i holds coef[B(i+2)][t]) and
// the B operand to the t-th term (I, A, A^2, A^3, A^6) of this lane's element,
// five MFMA steps leave B2..B5 of that element in the four accumulator VGPRs:
// the chain c0*I, +c1*A, +c2*A^2, +c3*A^3, +c6*A^6 of the reference's
// contracted combine (csrc/MatrixExpSmall.cuh:74-77).  B1 (used only as a left
// operand) is formed directly in transposed layout on the VALU.
//
// Per matrix everything is independent of the batch size and of the slot the
// matrix lands in (csrc tests demand bit-identical results across B).
#include "fh_kernels.h"

namespace fh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

struct Q {
  float v[4];
};

template <bool Pair>
struct PQ {
  Q d;
  Q u;
};

__device__ __forceinline__ float dpp_xor1(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_xor2(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ int dpp_xor1_i(int x) { return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int dpp_xor2_i(int x) { return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ double dpp_xor1_d(double x) {
  const int2 w = __builtin_bit_cast(int2, x);
  return __builtin_bit_cast(double, make_int2(dpp_xor1_i(w.x), dpp_xor1_i(w.y)));
}
__device__ __forceinline__ double dpp_xor2_d(double x) {
  const int2 w = __builtin_bit_cast(int2, x);
  return __builtin_bit_cast(double, make_int2(dpp_xor2_i(w.x), dpp_xor2_i(w.y)));
}

// In-quad transpose: lane j, v[r] = M[r][j]  ->  v[r] = M[j][r].  Two
// butterfly stages exchange (lane bit 0, VGPR bit 0) and (lane bit 1, VGPR bit 1).
__device__ __forceinline__ Q transpose(const Q& m, int j) {
  const bool odd = j & 1;
  const bool hi = j & 2;
  const float p0 = dpp_xor1(m.v[0]), p1 = dpp_xor1(m.v[1]), p2 = dpp_xor1(m.v[2]), p3 = dpp_xor1(m.v[3]);
  const float s0 = odd ? p1 : m.v[0];
  const float s1 = odd ? m.v[1] : p0;
  const float s2 = odd ? p3 : m.v[2];
  const float s3 = odd ? m.v[3] : p2;
  const float q0 = dpp_xor2(s0), q1 = dpp_xor2(s1), q2 = dpp_xor2(s2), q3 = dpp_xor2(s3);
  Q t;
  t.v[0] = hi ? q2 : s0;
  t.v[1] = hi ? q3 : s1;
  t.v[2] = hi ? s2 : q0;
  t.v[3] = hi ? s3 : q1;
  return t;
}

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

// C-layout of X.Y from (X^T, Y).
__device__ __forceinline__ Q mm(const Q& xt, const Q& y) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma4(xt.v[0], y.v[0], acc);
  acc = mfma4(xt.v[1], y.v[1], acc);
  acc = mfma4(xt.v[2], y.v[2], acc);
  acc = mfma4(xt.v[3], y.v[3], acc);
  return Q{{acc[0], acc[1], acc[2], acc[3]}};
}

// C-layout of (X.Y)^T from (X^T, Y).
__device__ __forceinline__ Q mmT(const Q& xt, const Q& y) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma4(y.v[0], xt.v[0], acc);
  acc = mfma4(y.v[1], xt.v[1], acc);
  acc = mfma4(y.v[2], xt.v[2], acc);
  acc = mfma4(y.v[3], xt.v[3], acc);
  return Q{{acc[0], acc[1], acc[2], acc[3]}};
}

__device__ __forceinline__ Q qadd(const Q& a, const Q& b) {
  return Q{{a.v[0] + b.v[0], a.v[1] + b.v[1], a.v[2] + b.v[2], a.v[3] + b.v[3]}};
}

__device__ __forceinline__ Q qsel(bool p, const Q& a, const Q& b) {
  return Q{{p ? a.v[0] : b.v[0], p ? a.v[1] : b.v[1], p ? a.v[2] : b.v[2], p ? a.v[3] : b.v[3]}};
}

// Structured (Frechet) product: (D1.D2, D1.U2 + U1.D2), the two U sums kept
// separate and added last (csrc/MatrixExpSmall.cuh:34-49).
template <bool Pair>
__device__ __forceinline__ PQ<Pair> pmm(const PQ<Pair>& xt, const PQ<Pair>& y) {
  PQ<Pair> c;
  c.d = mm(xt.d, y.d);
  if constexpr (Pair) c.u = qadd(mm(xt.d, y.u), mm(xt.u, y.d));
  return c;
}
template <bool Pair>
__device__ __forceinline__ PQ<Pair> pmmT(const PQ<Pair>& xt, const PQ<Pair>& y) {
  PQ<Pair> c;
  c.d = mmT(xt.d, y.d);
  if constexpr (Pair) c.u = qadd(mmT(xt.d, y.u), mmT(xt.u, y.d));
  return c;
}
template <bool Pair>
__device__ __forceinline__ PQ<Pair> padd(const PQ<Pair>& a, const PQ<Pair>& b) {
  PQ<Pair> c;
  c.d = qadd(a.d, b.d);
  if constexpr (Pair) c.u = qadd(a.u, b.u);
  return c;
}
template <bool Pair>
__device__ __forceinline__ PQ<Pair> ptranspose(const PQ<Pair>& a, int j) {
  PQ<Pair> c;
  c.d = transpose(a.d, j);
  if constexpr (Pair) c.u = transpose(a.u, j);
  return c;
}
template <bool Pair>
__device__ __forceinline__ PQ<Pair> psel(bool p, const PQ<Pair>& a, const PQ<Pair>& b) {
  PQ<Pair> c;
  c.d = qsel(p, a.d, b.d);
  if constexpr (Pair) c.u = qsel(p, a.u, b.u);
  return c;
}

// B1^T = c1*A^T + c2*(A^2)^T + c3*(A^3)^T (B1 has no I and no A^6 term).
__device__ __forceinline__ Q b1_transposed(const Q& at, const Q& a2t, const Q& a3t) {
  Q b;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float t = __builtin_fmaf(kCoef[0][1], at.v[r], 0.f);
    t = __builtin_fmaf(kCoef[0][2], a2t.v[r], t);
    b.v[r] = __builtin_fmaf(kCoef[0][3], a3t.v[r], t);
  }
  return b;
}

// B2..B5 on MFMA.  cf[t] holds coef[B(2 + lane%4)][t]; ident[r] is I[r][j].
// with_identity is false for the U blocks (the identity goes to D only).
__device__ __forceinline__ void combine_mfma(const float (&cf)[5], const float (&ident)[4], bool with_identity,
                                             const Q& a, const Q& a2, const Q& a3, const Q& a6, Q& b2, Q& b3, Q& b4,
                                             Q& b5) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (with_identity) acc = mfma4(cf[0], ident[r], acc);
    acc = mfma4(cf[1], a.v[r], acc);
    acc = mfma4(cf[2], a2.v[r], acc);
    acc = mfma4(cf[3], a3.v[r], acc);
    acc = mfma4(cf[4], a6.v[r], acc);
    b2.v[r] = acc[0];
    b3.v[r] = acc[1];
    b4.v[r] = acc[2];
    b5.v[r] = acc[3];
  }
}

// ---- loads / stores ---------------------------------------------------------

// v[r] = M[j][r] (row j of the logical matrix, zero padded to 4).
template <typename T>
__device__ __forceinline__ Q load_row(const Operand& op, int64_t b, int j, int n, bool valid) {
  Q q{{0.f, 0.f, 0.f, 0.f}};
  if (!valid || j >= n) return q;
  using S = typename T::storage;
  typedef S S4 __attribute__((ext_vector_type(4)));
  const S* p = static_cast<const S*>(op.data);
  if (op.vec == kVecRows) {
    const S4 w = *reinterpret_cast<const S4*>(p + b * op.sb + static_cast<int64_t>(j) * op.sr);
    q.v[0] = to_f32<T>(w[0]) * op.sign;
    q.v[1] = to_f32<T>(w[1]) * op.sign;
    q.v[2] = to_f32<T>(w[2]) * op.sign;
    q.v[3] = to_f32<T>(w[3]) * op.sign;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (r < n) q.v[r] = load_elem<T>(op, b, j, r);
  }
  return q;
}

// v[r] = M[r][j] (column j of the logical matrix, zero padded to 4).
template <typename T>
__device__ __forceinline__ Q load_col(const Operand& op, int64_t b, int j, int n, bool valid) {
  Q q{{0.f, 0.f, 0.f, 0.f}};
  if (!valid || j >= n) return q;
  using S = typename T::storage;
  typedef S S4 __attribute__((ext_vector_type(4)));
  const S* p = static_cast<const S*>(op.data);
  if (op.vec == kVecCols) {
    const S4 w = *reinterpret_cast<const S4*>(p + b * op.sb + static_cast<int64_t>(j) * op.sc);
    q.v[0] = to_f32<T>(w[0]) * op.sign;
    q.v[1] = to_f32<T>(w[1]) * op.sign;
    q.v[2] = to_f32<T>(w[2]) * op.sign;
    q.v[3] = to_f32<T>(w[3]) * op.sign;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (r < n) q.v[r] = load_elem<T>(op, b, r, j);
  }
  return q;
}

// Writes row j of the result from its transposed C-layout (v[r] = M[j][r]).
template <typename T>
__device__ __forceinline__ void store_row(void* out, int64_t b, int j, int n, const Q& rowv) {
  using S = typename T::storage;
  S* p = static_cast<S*>(out) + (b * n + j) * n;
  if (n == 4) {
    typedef S S4 __attribute__((ext_vector_type(4)));
    S4 w;
    w[0] = from_f32<T>(rowv.v[0]);
    w[1] = from_f32<T>(rowv.v[1]);
    w[2] = from_f32<T>(rowv.v[2]);
    w[3] = from_f32<T>(rowv.v[3]);
    *reinterpret_cast<S4*>(p) = w;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (r < n) p[r] = from_f32<T>(rowv.v[r]);
  }
}

constexpr int kQuadWaves = 4;  // wavefronts per workgroup

template <typename T, bool Pair>
__global__ __launch_bounds__(64 * kQuadWaves) void expm_quad_kernel(ExpmArgs args) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane & 3;
  const int n = args.n;
  const int64_t b = (static_cast<int64_t>(blockIdx.x) * kQuadWaves + wave) * 16 + (lane >> 2);
  const bool valid = b < args.batch;

  // Coefficient column of this lane for the B2..B5 MFMA, and I[r][j].
  float cf[5];
#pragma unroll
  for (int t = 0; t < 5; ++t) cf[t] = (j == 0) ? kCoef[1][t] : (j == 1) ? kCoef[2][t] : (j == 2) ? kCoef[3][t] : kCoef[4][t];
  float ident[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) ident[r] = (r == j) ? 1.f : 0.f;

  PQ<Pair> a, at;
  a.d = load_col<T>(args.x, b, j, n, valid);
  at.d = load_row<T>(args.x, b, j, n, valid);
  bool bad = false;
#pragma unroll
  for (int r = 0; r < 4; ++r) bad |= !finite_f32(a.d.v[r]);
  if constexpr (Pair) {
    a.u = load_col<T>(args.g, b, j, n, valid);
    at.u = load_row<T>(args.g, b, j, n, valid);
#pragma unroll
    for (int r = 0; r < 4; ++r) bad |= !finite_f32(a.u.v[r]);
  }
  // Non-finite rule over the whole matrix (csrc/MatrixExpSmall.cuh:126-140).
  int badq = bad ? 1 : 0;
  badq |= dpp_xor1_i(badq);
  badq |= dpp_xor2_i(badq);

  // FP64 1-norm: this lane owns column j; rows combine as ((x0+x2)+(x1+x3))
  // (the lane butterfly of csrc/MatrixExpSmall.cuh:146-152).
  double x[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    x[r] = fabs(static_cast<double>(a.d.v[r]));
    if constexpr (Pair) x[r] += fabs(static_cast<double>(a.u.v[r]));
  }
  const double col = (x[0] + x[2]) + (x[1] + x[3]);
  double norm = fmax(col, dpp_xor1_d(col));
  norm = fmax(norm, dpp_xor2_d(norm));
  const int s = badq ? 0 : squarings_from_norm(norm);

  const float scale = __builtin_ldexpf(1.f, -s);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    a.d.v[r] *= scale;
    at.d.v[r] *= scale;
    if constexpr (Pair) {
      a.u.v[r] *= scale;
      at.u.v[r] *= scale;
    }
  }

  // Degree-18 polynomial in the reference's product order
  // (csrc/MatrixExpSmall.cuh:86-105): A2 = A.A, A3 = A2.A, A6 = A3.A3.
  const PQ<Pair> a2 = pmm<Pair>(at, a);
  const PQ<Pair> a2t = pmmT<Pair>(at, a);
  const PQ<Pair> a3 = pmm<Pair>(a2t, a);
  const PQ<Pair> a3t = pmmT<Pair>(a2t, a);
  const PQ<Pair> a6 = pmm<Pair>(a3t, a3);
  PQ<Pair> b1t, b2, b3, b4, b5;
  b1t.d = b1_transposed(at.d, a2t.d, a3t.d);
  combine_mfma(cf, ident, true, a.d, a2.d, a3.d, a6.d, b2.d, b3.d, b4.d, b5.d);
  if constexpr (Pair) {
    b1t.u = b1_transposed(at.u, a2t.u, a3t.u);
    combine_mfma(cf, ident, false, a.u, a2.u, a3.u, a6.u, b2.u, b3.u, b4.u, b5.u);
  }
  // A9 = B1.B5 + B4; T = B2 + (B3 + A9).A9.
  const PQ<Pair> a9 = padd<Pair>(pmm<Pair>(b1t, b5), b4);
  const PQ<Pair> lhs_t = ptranspose<Pair>(padd<Pair>(b3, a9), j);
  PQ<Pair> res = padd<Pair>(b2, pmm<Pair>(lhs_t, a9));

  // s squarings per matrix (csrc/MatrixExpSmall.cuh:168); the wavefront runs
  // to its largest s and each matrix keeps its own result.
  int smax = s;
#pragma unroll
  for (int off = 4; off < 64; off <<= 1) smax = max(smax, __shfl_xor(smax, off));
  smax = __builtin_amdgcn_readfirstlane(smax);
  PQ<Pair> rest = ptranspose<Pair>(res, j);
  for (int i = 0; i < smax; ++i) {
    const bool keep = i < s;
    const PQ<Pair> nxt = pmm<Pair>(rest, res);
    const PQ<Pair> nxtt = pmmT<Pair>(rest, res);
    res = psel<Pair>(keep, nxt, res);
    rest = psel<Pair>(keep, nxtt, rest);
  }

  if (valid && j < n) {
    Q rowv = Pair ? rest.u : rest.d;
    if (badq) {
#pragma unroll
      for (int r = 0; r < 4; ++r) rowv.v[r] = __builtin_nanf("");
    }
    store_row<T>(args.out, b, j, n, rowv);
  }
  if (valid && j == 0 && args.s_out) args.s_out[b] = badq ? -1 : s;
}

template <typename T, bool Pair>
hipError_t launch_quad_t(const ExpmArgs& args, hipStream_t stream) {
  const int64_t per_block = 16 * kQuadWaves;
  const int64_t grid = (args.batch + per_block - 1) / per_block;
  hipLaunchKernelGGL((expm_quad_kernel<T, Pair>), dim3(static_cast<unsigned>(grid)), dim3(64 * kQuadWaves), 0,
                     stream, args);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quad(const ExpmArgs& args, int dtype, bool pair, hipStream_t stream) {
  if (dtype == F32::code) return pair ? launch_quad_t<F32, true>(args, stream) : launch_quad_t<F32, false>(args, stream);
  if (dtype == BF16::code) return pair ? launch_quad_t<BF16, true>(args, stream) : launch_quad_t<BF16, false>(args, stream);
  return pair ? launch_quad_t<F16, true>(args, stream) : launch_quad_t<F16, false>(args, stream);
}

}  // namespace fh

// Per-lane pieces of the P == 4 kernels (n = 2, 3, 4), shared by the matrix
// exponential (expm_p4.hip) and the fused hyper-connection stream mixing
// (hc_mix.hip): one matrix per lane, held in registers as a row-major 4 x 4
// (FP32), or as a (D, U) pair for the Frechet derivative.
//
// Arithmetic is the reference's, element by element (csrc/MatrixExpSmall.cuh:
// 22-106): product entries accumulate k = 0..3 with fmaf from +0, Frechet U
// blocks sum D.U and U.D separately and add them, combines are the
// contracted chain c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 with its zero
// coefficients skipped.  Results are bit-identical to that evaluation up to
// the sign of zero results.
#pragma once

#include "fh_kernels.h"

namespace fh {
namespace p4 {

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

// Compiler ordering of the wavefront's LDS accesses (the hardware performs
// one wavefront's LDS operations in issue order).
__device__ __forceinline__ void lds_order() {
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_sched_barrier(0);
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

}  // namespace p4
}  // namespace fh

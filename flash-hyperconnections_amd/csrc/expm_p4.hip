// P == 4 kernel (n = 2, 3, 4): one matrix per lane, 64 matrices per
// wavefront.
//
// Each lane keeps its whole 4 x 4 matrix (16 VGPRs; the Frechet kernel keeps
// the D and U blocks, 32 VGPRs) and every product is 64 plain FP32 FMAs with
// compile-time register indices -- no cross-lane traffic, no transposes.  On
// gfx950 a 64-lane FP32 FMA issues every 2 cycles (the same rate as the 4x4x1
// MFMA, which cannot overlap with VALU work), while DPP-sourced operands run
// at half rate, so this layout is the one that reaches the FMA floor.  The
// per-matrix scalar work (FP64 norm, squaring count, scaling) is also done
// once per matrix rather than once per row.
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

// Row i of X.Y into c (four entries, k = 0..3 in order).
__device__ __forceinline__ void mul_row(const M4& x, const M4& y, int i, float* c) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float acc = __builtin_fmaf(x.v[4 * i], y.v[j], 0.f);
    acc = __builtin_fmaf(x.v[4 * i + 1], y.v[4 + j], acc);
    acc = __builtin_fmaf(x.v[4 * i + 2], y.v[8 + j], acc);
    c[j] = __builtin_fmaf(x.v[4 * i + 3], y.v[12 + j], acc);
  }
}

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

// The whole pipeline for the matrix of this lane.
template <typename T, bool Pair, int XL>
__device__ __forceinline__ void compute_matrix(const ExpmArgs& args, PM<Pair> a, int64_t b, int n, bool valid,
                                               int lane, bool full_group, float* tile) {
  // FP64 1-norm: column sums over rows as ((x0 + x2) + (x1 + x3)) with
  // x_r = |A[r][j]| (+ |G[r][j]|), the reference's butterfly order
  // (csrc/MatrixExpSmall.cuh:144-152).  The sum of the column sums is finite
  // exactly when every entry is: the non-finite rule of
  // csrc/MatrixExpSmall.cuh:126-140.
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
  const bool bad = !__builtin_isfinite(total);
  const int s = bad ? 0 : squarings_from_norm(norm);

  // Scale by 2^-s (csrc/MatrixExpSmall.cuh:157-162) with the views' lazy
  // negation folded into the same exact multiply.
  const float scale = __builtin_ldexpf(1.f, -s);
  const float scale_x = scale * args.x.sign;
  const float scale_g = scale * args.g.sign;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    a.d.v[e] *= scale_x;
    if constexpr (Pair) a.u.v[e] *= scale_g;
  }

  // Degree-18 polynomial (csrc/MatrixExpSmall.cuh:83-106):
  // A2 = A.A, A3 = A2.A, A6 = A3.A3, A9 = B1.B5 + B4, T = B2 + (B3 + A9).A9.
  const PM<Pair> a2 = pmul<Pair>(a, a);
  const PM<Pair> a3 = pmul<Pair>(a2, a);
  const PM<Pair> a6 = pmul<Pair>(a3, a3);
  PM<Pair> a9;
  {
    const PM<Pair> b5 = comb<4, Pair>(a, a2, a3, a6);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // B1 one row at a time
      float b1d[4], b1u[4], b4d[4], b4u[4];
      comb_row<0, Pair>(a, a2, a3, a6, i, b1d, b1u);
      pmul_row<Pair>(b1d, b1u, b5, &a9.d.v[4 * i], &a9.u.v[4 * i]);
      comb_row<3, Pair>(a, a2, a3, a6, i, b4d, b4u);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a9.d.v[4 * i + j] += b4d[j];
        if constexpr (Pair) a9.u.v[4 * i + j] += b4u[j];
      }
    }
  }
  PM<Pair> res;
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // (B3 + A9) and B2 one row at a time
    float ld[4], lu[4], b2d[4], b2u[4], qd[4], qu[4];
    comb_row<2, Pair>(a, a2, a3, a6, i, ld, lu);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ld[j] += a9.d.v[4 * i + j];
      if constexpr (Pair) lu[j] += a9.u.v[4 * i + j];
    }
    pmul_row<Pair>(ld, lu, a9, qd, qu);
    comb_row<1, Pair>(a, a2, a3, a6, i, b2d, b2u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      res.d.v[4 * i + j] = b2d[j] + qd[j];
      if constexpr (Pair) res.u.v[4 * i + j] = b2u[j] + qu[j];
    }
  }

  // s squarings per matrix (csrc/MatrixExpSmall.cuh:168); the wavefront loops
  // while any of its matrices still needs one and each keeps its own result.
  for (int it = 0; __builtin_amdgcn_ballot_w64(it < s) != 0; ++it) {
    const PM<Pair> sq = pmul<Pair>(res, res);
    const bool keep = it < s;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      res.d.v[e] = keep ? sq.d.v[e] : res.d.v[e];
      if constexpr (Pair) res.u.v[e] = keep ? sq.u.v[e] : res.u.v[e];
    }
  }

  M4 outm = Pair ? res.u : res.d;
  if (bad) {
#pragma unroll
    for (int e = 0; e < 16; ++e) outm.v[e] = __builtin_nanf("");
  }
  if constexpr (XL != kVecNone) {
    if (full_group) {
      store_group_staged<T>(args.out, b - lane, lane, outm, tile);
    } else if (valid) {
      store_matrix<T, true>(args.out, b, n, outm);
    }
  } else {
    if (valid) store_matrix<T, false>(args.out, b, n, outm);
  }
  if (valid && args.s_out) args.s_out[b] = bad ? -1 : s;
}

// Persistent kernel: each wavefront walks 64-matrix groups with a grid stride
// and issues the loads of its next group before computing the current one, so
// HBM latency overlaps the arithmetic of the previous group.
template <typename T, bool Pair, int XL, int GL>
__global__ __launch_bounds__(64 * kP4Waves) void expm_p4_kernel(ExpmArgs args) {
  __shared__ float stage[kP4Waves][64 * kStageStride];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = (XL != kVecNone) ? 4 : args.n;
  const int64_t groups = (args.batch + 63) / 64;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kP4Waves;
  int64_t group = static_cast<int64_t>(blockIdx.x) * kP4Waves + wave;

  PM<Pair> next;
  if (group < groups) {
    const int64_t b = group * 64 + lane;
    next.d = load_matrix<T, XL>(args.x, b, n, b < args.batch);
    if constexpr (Pair) next.u = load_matrix<T, GL>(args.g, b, n, b < args.batch);
  }
  for (; group < groups; group += stride) {
    const PM<Pair> cur = next;
    const int64_t b = group * 64 + lane;
    if (group + stride < groups) {
      const int64_t nb = (group + stride) * 64 + lane;
      next.d = load_matrix<T, XL>(args.x, nb, n, nb < args.batch);
      if constexpr (Pair) next.u = load_matrix<T, GL>(args.g, nb, n, nb < args.batch);
    }
    const bool full_group = (group + 1) * 64 <= args.batch;
    compute_matrix<T, Pair, XL>(args, cur, b, n, b < args.batch, lane, full_group, stage[wave]);
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

// P in {16, 32} kernel (n = 9..32): one 64-lane wavefront per matrix, every
// product on FP32 MFMA (v_mfma_f32_16x16x4_f32 for P = 16,
// v_mfma_f32_32x32x2_f32 for P = 32).
//
// Layout: a P x P matrix occupies R = P*P/64 VGPRs per lane in the MFMA
// accumulator ("D") layout: lane l, VGPR r holds M[row(l, r)][l % P] with
//   P = 16: row = 4*(l/16) + r
//   P = 32: row = 8*(r/4) + 4*(l/32) + r%4.
// Step r of a product feeds the A operand from VGPR r of X^T and the B operand
// from VGPR r of Y; lane group g then contributes k = row(g, r), so the R
// steps together cover k = 0..P-1 and
//   X.Y = sum_r mfma(a = (X^T).v[r], b = Y.v[r])
// needs no data movement for Y.  Left operands are transposed through a
// padded LDS tile (P x (P+1) floats).  The kernel is MFMA-bound, so the
// polynomial's combines stay on the otherwise idle VALU.
#include "fh_kernels.h"

namespace fh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

template <int P>
struct TileCfg;

template <>
struct TileCfg<16> {
  static constexpr int R = 4;
  using acc_t = v4f;
  __device__ static __forceinline__ int row(int lane, int r) { return 4 * (lane >> 4) + r; }
  __device__ static __forceinline__ int col(int lane) { return lane & 15; }
  __device__ static __forceinline__ acc_t mfma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

template <>
struct TileCfg<32> {
  static constexpr int R = 16;
  using acc_t = v16f;
  __device__ static __forceinline__ int row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
  __device__ static __forceinline__ int col(int lane) { return lane & 31; }
  __device__ static __forceinline__ acc_t mfma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

template <int P>
struct Tm {
  float v[TileCfg<P>::R];
};

template <int P, bool Pair>
struct PTm {
  Tm<P> d;
  Tm<P> u;
};

template <int P>
__device__ __forceinline__ Tm<P> mm(const Tm<P>& xt, const Tm<P>& y) {
  using C = TileCfg<P>;
  typename C::acc_t acc = {};
#pragma unroll
  for (int r = 0; r < C::R; ++r) acc = C::mfma(xt.v[r], y.v[r], acc);
  Tm<P> out;
#pragma unroll
  for (int r = 0; r < C::R; ++r) out.v[r] = acc[r];
  return out;
}

template <int P>
__device__ __forceinline__ Tm<P> tadd(const Tm<P>& a, const Tm<P>& b) {
  Tm<P> c;
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) c.v[r] = a.v[r] + b.v[r];
  return c;
}

// D-layout of M -> D-layout of M^T through the wavefront's LDS tile.  The
// workgroup is this one wavefront, so the barriers only order its own LDS
// traffic.
template <int P>
__device__ __forceinline__ Tm<P> transpose(const Tm<P>& m, float* buf, int lane) {
  using C = TileCfg<P>;
  constexpr int LD = P + 1;
  const int c = C::col(lane);
#pragma unroll
  for (int r = 0; r < C::R; ++r) buf[C::row(lane, r) * LD + c] = m.v[r];
  __syncthreads();
  Tm<P> t;
#pragma unroll
  for (int r = 0; r < C::R; ++r) t.v[r] = buf[c * LD + C::row(lane, r)];
  __syncthreads();
  return t;
}

template <int P, bool Pair>
__device__ __forceinline__ PTm<P, Pair> pmm(const PTm<P, Pair>& xt, const PTm<P, Pair>& y) {
  PTm<P, Pair> c;
  c.d = mm<P>(xt.d, y.d);
  if constexpr (Pair) c.u = tadd<P>(mm<P>(xt.d, y.u), mm<P>(xt.u, y.d));
  return c;
}
template <int P, bool Pair>
__device__ __forceinline__ PTm<P, Pair> padd(const PTm<P, Pair>& a, const PTm<P, Pair>& b) {
  PTm<P, Pair> c;
  c.d = tadd<P>(a.d, b.d);
  if constexpr (Pair) c.u = tadd<P>(a.u, b.u);
  return c;
}
template <int P, bool Pair>
__device__ __forceinline__ PTm<P, Pair> ptranspose(const PTm<P, Pair>& a, float* buf, int lane) {
  PTm<P, Pair> c;
  c.d = transpose<P>(a.d, buf, lane);
  if constexpr (Pair) c.u = transpose<P>(a.u, buf, lane);
  return c;
}

// B(k+1) = c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 as the reference's
// contracted chain (csrc/MatrixExpSmall.cuh:268-281); identity on D only.
template <int P, bool Pair>
__device__ __forceinline__ PTm<P, Pair> combine(const PTm<P, Pair>& a, const PTm<P, Pair>& a2,
                                                const PTm<P, Pair>& a3, const PTm<P, Pair>& a6, int k,
                                                const float (&diag)[TileCfg<P>::R]) {
  PTm<P, Pair> b;
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) {
    float t = kCoef[k][0] * diag[r];
    t = __builtin_fmaf(kCoef[k][1], a.d.v[r], t);
    t = __builtin_fmaf(kCoef[k][2], a2.d.v[r], t);
    t = __builtin_fmaf(kCoef[k][3], a3.d.v[r], t);
    b.d.v[r] = __builtin_fmaf(kCoef[k][4], a6.d.v[r], t);
    if constexpr (Pair) {
      float w = kCoef[k][1] * a.u.v[r];
      w = __builtin_fmaf(kCoef[k][2], a2.u.v[r], w);
      w = __builtin_fmaf(kCoef[k][3], a3.u.v[r], w);
      b.u.v[r] = __builtin_fmaf(kCoef[k][4], a6.u.v[r], w);
    }
  }
  return b;
}

template <typename T, int P, bool Pair>
__global__ __launch_bounds__(64) void expm_tile_kernel(ExpmArgs args) {
  using C = TileCfg<P>;
  constexpr int R = C::R;
  constexpr int LD = P + 1;
  __shared__ float buf[2 * P * LD];
  __shared__ double colsum[P];
  const int lane = threadIdx.x;
  const int c = C::col(lane);
  const int n = args.n;
  float diag[R];
#pragma unroll
  for (int r = 0; r < R; ++r) diag[r] = (C::row(lane, r) == c) ? 1.f : 0.f;

  for (int64_t b = blockIdx.x; b < args.batch; b += gridDim.x) {
    PTm<P, Pair> a, at;
    bool bad = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = C::row(lane, r);
      const bool in = row < n && c < n;
      a.d.v[r] = in ? load_elem<T>(args.x, b, row, c) : 0.f;
      at.d.v[r] = in ? load_elem<T>(args.x, b, c, row) : 0.f;
      bad |= !finite_f32(a.d.v[r]);
      if constexpr (Pair) {
        a.u.v[r] = in ? load_elem<T>(args.g, b, row, c) : 0.f;
        at.u.v[r] = in ? load_elem<T>(args.g, b, c, row) : 0.f;
        bad |= !finite_f32(a.u.v[r]);
      }
    }
    // Non-finite rule (csrc/MatrixExpSmall.cuh:318-331).
    if (__syncthreads_or(bad)) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = C::row(lane, r);
        if (row < n && c < n) store_elem<T>(args.out, (b * n + row) * n + c, __builtin_nanf(""));
      }
      if (lane == 0 && args.s_out) args.s_out[b] = -1;
      continue;
    }
    // FP64 1-norm, rows summed sequentially per column, |A| then |G| per row
    // (csrc/MatrixExpSmall.cuh:343-357).
#pragma unroll
    for (int r = 0; r < R; ++r) {
      buf[C::row(lane, r) * LD + c] = a.d.v[r];
      if constexpr (Pair) buf[P * LD + C::row(lane, r) * LD + c] = a.u.v[r];
    }
    __syncthreads();
    if (lane < P) {
      double v = 0.;
      for (int row = 0; row < P; ++row) {
        v += fabs(static_cast<double>(buf[row * LD + lane]));
        if constexpr (Pair) v += fabs(static_cast<double>(buf[P * LD + row * LD + lane]));
      }
      colsum[lane] = v;
    }
    __syncthreads();
    double norm = 0.;
    for (int j = 0; j < P; ++j) norm = fmax(norm, colsum[j]);
    const int s = squarings_from_norm(norm);
    __syncthreads();

    const float scale = __builtin_ldexpf(1.f, -s);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      a.d.v[r] *= scale;
      at.d.v[r] *= scale;
      if constexpr (Pair) {
        a.u.v[r] *= scale;
        at.u.v[r] *= scale;
      }
    }
    // Degree-18 polynomial.  Powers are formed as A.A and A.A^2 (all factors
    // are polynomials in the same matrix), then A^6 = A^3.A^3, A9 = B1.B5 + B4,
    // T = B2 + (B3 + A9).A9.
    const PTm<P, Pair> a2 = pmm<P, Pair>(at, a);
    const PTm<P, Pair> a3 = pmm<P, Pair>(at, a2);
    const PTm<P, Pair> a6 = pmm<P, Pair>(ptranspose<P, Pair>(a3, buf, lane), a3);
    const PTm<P, Pair> b1t = ptranspose<P, Pair>(combine<P, Pair>(a, a2, a3, a6, 0, diag), buf, lane);
    const PTm<P, Pair> b5 = combine<P, Pair>(a, a2, a3, a6, 4, diag);
    const PTm<P, Pair> a9 = padd<P, Pair>(pmm<P, Pair>(b1t, b5), combine<P, Pair>(a, a2, a3, a6, 3, diag));
    const PTm<P, Pair> lhst =
        ptranspose<P, Pair>(padd<P, Pair>(combine<P, Pair>(a, a2, a3, a6, 2, diag), a9), buf, lane);
    const PTm<P, Pair> b2 = combine<P, Pair>(a, a2, a3, a6, 1, diag);
    PTm<P, Pair> res = padd<P, Pair>(b2, pmm<P, Pair>(lhst, a9));
    for (int i = 0; i < s; ++i) res = pmm<P, Pair>(ptranspose<P, Pair>(res, buf, lane), res);

#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = C::row(lane, r);
      if (row < n && c < n) store_elem<T>(args.out, (b * n + row) * n + c, Pair ? res.u.v[r] : res.d.v[r]);
    }
    if (lane == 0 && args.s_out) args.s_out[b] = s;
  }
}

template <typename T, int P, bool Pair>
hipError_t launch_tile_tp(const ExpmArgs& args, hipStream_t stream) {
  const int64_t grid = args.batch < (int64_t(1) << 30) ? args.batch : (int64_t(1) << 30);
  hipLaunchKernelGGL((expm_tile_kernel<T, P, Pair>), dim3(static_cast<unsigned>(grid)), dim3(64), 0, stream, args);
  return hipGetLastError();
}

template <typename T, bool Pair>
hipError_t launch_tile_t(const ExpmArgs& args, int P, hipStream_t stream) {
  return P == 16 ? launch_tile_tp<T, 16, Pair>(args, stream) : launch_tile_tp<T, 32, Pair>(args, stream);
}

}  // namespace

hipError_t launch_tile(const ExpmArgs& args, int dtype, int P, bool pair, hipStream_t stream) {
  if (dtype == F32::code) return pair ? launch_tile_t<F32, true>(args, P, stream) : launch_tile_t<F32, false>(args, P, stream);
  if (dtype == BF16::code) return pair ? launch_tile_t<BF16, true>(args, P, stream) : launch_tile_t<BF16, false>(args, P, stream);
  return pair ? launch_tile_t<F16, true>(args, P, stream) : launch_tile_t<F16, false>(args, P, stream);
}

}  // namespace fh

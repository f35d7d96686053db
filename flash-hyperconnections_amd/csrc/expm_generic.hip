// Generic kernel: one 64-lane wavefront per matrix, P x P tile (P = 4, 8, 16,
// 32), every product staged through LDS and accumulated per element with
// sequential fmaf over k.  It follows the reference's evaluation order exactly
// (csrc/MatrixExpSmall.cuh:22-106, :283-299) and is kept as a bit-exact
// checking aid for the tuned kernels, not as a fast path.
#include "fh_kernels.h"

namespace fh {
namespace {

template <int P, bool Pair>
struct GTile {
  static constexpr int E = (P * P + 63) / 64;  // elements owned per lane
  float d[E];
  float u[Pair ? E : 1];
};

template <int P, bool Pair>
__device__ __forceinline__ GTile<P, Pair> g_product(const GTile<P, Pair>& x, const GTile<P, Pair>& y, float* lds,
                                                    int lane) {
  constexpr int PP = P * P;
  constexpr int E = GTile<P, Pair>::E;
#pragma unroll
  for (int t = 0; t < E; ++t) {
    const int e = lane + 64 * t;
    if (e < PP) {
      lds[e] = x.d[t];
      lds[PP + e] = y.d[t];
      if constexpr (Pair) {
        lds[2 * PP + e] = x.u[t];
        lds[3 * PP + e] = y.u[t];
      }
    }
  }
  __syncthreads();
  GTile<P, Pair> c;
#pragma unroll
  for (int t = 0; t < E; ++t) {
    const int e = lane + 64 * t;
    c.d[t] = 0.f;
    if constexpr (Pair) c.u[t] = 0.f;
    if (e < PP) {
      const int i = e / P, j = e % P;
      float d = 0.f, u = 0.f, v = 0.f;
      for (int k = 0; k < P; ++k) {
        d = __builtin_fmaf(lds[i * P + k], lds[PP + k * P + j], d);
        if constexpr (Pair) u = __builtin_fmaf(lds[i * P + k], lds[3 * PP + k * P + j], u);
      }
      c.d[t] = d;
      if constexpr (Pair) {
        for (int k = 0; k < P; ++k) v = __builtin_fmaf(lds[2 * PP + i * P + k], lds[PP + k * P + j], v);
        c.u[t] = u + v;
      }
    }
  }
  __syncthreads();
  return c;
}

template <int P, bool Pair>
__device__ __forceinline__ GTile<P, Pair> g_add(const GTile<P, Pair>& a, const GTile<P, Pair>& b) {
  GTile<P, Pair> c;
#pragma unroll
  for (int t = 0; t < GTile<P, Pair>::E; ++t) {
    c.d[t] = a.d[t] + b.d[t];
    if constexpr (Pair) c.u[t] = a.u[t] + b.u[t];
  }
  return c;
}

// c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 as the FMA chain of the reference's
// contracted expression (csrc/MatrixExpSmall.cuh:74-77).
template <int P, bool Pair>
__device__ __forceinline__ GTile<P, Pair> g_combine(const GTile<P, Pair>& a, const GTile<P, Pair>& a2,
                                                    const GTile<P, Pair>& a3, const GTile<P, Pair>& a6, int row,
                                                    int lane) {
  GTile<P, Pair> b;
#pragma unroll
  for (int t = 0; t < GTile<P, Pair>::E; ++t) {
    const int e = lane + 64 * t;
    const float diag = ((e / P) == (e % P) && e < P * P) ? 1.f : 0.f;
    float v = kCoef[row][0] * diag;
    v = __builtin_fmaf(kCoef[row][1], a.d[t], v);
    v = __builtin_fmaf(kCoef[row][2], a2.d[t], v);
    v = __builtin_fmaf(kCoef[row][3], a3.d[t], v);
    v = __builtin_fmaf(kCoef[row][4], a6.d[t], v);
    b.d[t] = v;
    if constexpr (Pair) {
      float w = kCoef[row][1] * a.u[t];
      w = __builtin_fmaf(kCoef[row][2], a2.u[t], w);
      w = __builtin_fmaf(kCoef[row][3], a3.u[t], w);
      w = __builtin_fmaf(kCoef[row][4], a6.u[t], w);
      b.u[t] = w;
    }
  }
  return b;
}

template <typename T, int P, bool Pair>
__global__ __launch_bounds__(64) void expm_generic_kernel(ExpmArgs args) {
  constexpr int PP = P * P;
  constexpr int E = GTile<P, Pair>::E;
  __shared__ float lds[(Pair ? 4 : 2) * PP];
  __shared__ double colsum[P];
  const int lane = threadIdx.x;
  const int n = args.n;
  for (int64_t b = blockIdx.x; b < args.batch; b += gridDim.x) {
    GTile<P, Pair> a;
    bool bad = false;
#pragma unroll
    for (int t = 0; t < E; ++t) {
      const int e = lane + 64 * t;
      const int r = e / P, c = e % P;
      float v = 0.f, w = 0.f;
      if (e < PP && r < n && c < n) {
        v = load_elem<T>(args.x, b, r, c);
        if constexpr (Pair) w = load_elem<T>(args.g, b, r, c);
      }
      a.d[t] = v;
      bad |= !finite_f32(v);
      if constexpr (Pair) {
        a.u[t] = w;
        bad |= !finite_f32(w);
      }
    }
    // Non-finite rule (csrc/MatrixExpSmall.cuh:318-331).
    if (__syncthreads_or(bad)) {
#pragma unroll
      for (int t = 0; t < E; ++t) {
        const int e = lane + 64 * t;
        const int r = e / P, c = e % P;
        if (e < PP && r < n && c < n) store_elem<T>(args.out, (b * n + r) * n + c, __builtin_nanf(""));
      }
      if (lane == 0 && args.s_out) args.s_out[b] = -1;
      continue;
    }
    // FP64 1-norm with the reference's association per P.
#pragma unroll
    for (int t = 0; t < E; ++t) {
      const int e = lane + 64 * t;
      if (e < PP) {
        lds[e] = a.d[t];
        if constexpr (Pair) lds[PP + e] = a.u[t];
      }
    }
    __syncthreads();
    if (lane < P) {
      const int j = lane;
      double col;
      if constexpr (P <= 8) {
        double x[P];
#pragma unroll
        for (int r = 0; r < P; ++r) {
          x[r] = fabs(static_cast<double>(lds[r * P + j]));
          if constexpr (Pair) x[r] += fabs(static_cast<double>(lds[PP + r * P + j]));
        }
        if constexpr (P == 4) {
          col = (x[0] + x[2]) + (x[1] + x[3]);
        } else {
          col = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
        }
      } else {
        col = 0.;
        for (int r = 0; r < P; ++r) {
          col += fabs(static_cast<double>(lds[r * P + j]));
          if constexpr (Pair) col += fabs(static_cast<double>(lds[PP + r * P + j]));
        }
      }
      colsum[j] = col;
    }
    __syncthreads();
    double norm = 0.;
    for (int j = 0; j < P; ++j) norm = fmax(norm, colsum[j]);
    const int s = squarings_from_norm(norm);
    __syncthreads();
    const float scale = __builtin_ldexpf(1.f, -s);
#pragma unroll
    for (int t = 0; t < E; ++t) {
      a.d[t] *= scale;
      if constexpr (Pair) a.u[t] *= scale;
    }
    // Degree-18 polynomial (csrc/MatrixExpSmall.cuh:283-299).
    auto a2 = g_product<P, Pair>(a, a, lds, lane);
    auto a3 = g_product<P, Pair>(a2, a, lds, lane);
    auto a6 = g_product<P, Pair>(a3, a3, lds, lane);
    auto b1 = g_combine<P, Pair>(a, a2, a3, a6, 0, lane);
    auto b2 = g_combine<P, Pair>(a, a2, a3, a6, 1, lane);
    auto b3 = g_combine<P, Pair>(a, a2, a3, a6, 2, lane);
    auto b4 = g_combine<P, Pair>(a, a2, a3, a6, 3, lane);
    auto b5 = g_combine<P, Pair>(a, a2, a3, a6, 4, lane);
    auto a9 = g_add<P, Pair>(g_product<P, Pair>(b1, b5, lds, lane), b4);
    auto res = g_add<P, Pair>(b2, g_product<P, Pair>(g_add<P, Pair>(b3, a9), a9, lds, lane));
    for (int i = 0; i < s; ++i) res = g_product<P, Pair>(res, res, lds, lane);
#pragma unroll
    for (int t = 0; t < E; ++t) {
      const int e = lane + 64 * t;
      const int r = e / P, c = e % P;
      if (e < PP && r < n && c < n) store_elem<T>(args.out, (b * n + r) * n + c, Pair ? res.u[t] : res.d[t]);
    }
    if (lane == 0 && args.s_out) args.s_out[b] = s;
  }
}

template <typename T, int P, bool Pair>
hipError_t launch_generic_tp(const ExpmArgs& args, hipStream_t stream) {
  const int64_t grid = args.batch < (int64_t(1) << 30) ? args.batch : (int64_t(1) << 30);
  hipLaunchKernelGGL((expm_generic_kernel<T, P, Pair>), dim3(static_cast<unsigned>(grid)), dim3(64), 0, stream,
                     args);
  return hipGetLastError();
}

template <typename T, bool Pair>
hipError_t launch_generic_t(const ExpmArgs& args, int P, hipStream_t stream) {
  switch (P) {
    case 4: return launch_generic_tp<T, 4, Pair>(args, stream);
    case 8: return launch_generic_tp<T, 8, Pair>(args, stream);
    case 16: return launch_generic_tp<T, 16, Pair>(args, stream);
    default: return launch_generic_tp<T, 32, Pair>(args, stream);
  }
}

}  // namespace

hipError_t launch_generic(const ExpmArgs& args, int dtype, int P, bool pair, hipStream_t stream) {
  if (dtype == F32::code) return pair ? launch_generic_t<F32, true>(args, P, stream) : launch_generic_t<F32, false>(args, P, stream);
  if (dtype == BF16::code) return pair ? launch_generic_t<BF16, true>(args, P, stream) : launch_generic_t<BF16, false>(args, P, stream);
  return pair ? launch_generic_t<F16, true>(args, P, stream) : launch_generic_t<F16, false>(args, P, stream);
}

}  // namespace fh

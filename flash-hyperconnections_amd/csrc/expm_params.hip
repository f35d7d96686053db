// Selection parameters only: one thread per matrix computes the FP64 1-norm
// with the association the main kernels use for its padded size P and the
// squaring count from it (reference csrc/MatrixExpSmall.cuh:141-154, :332-361).
#include "fh_kernels.h"

namespace fh {
namespace {

template <typename T, int P, bool Pair>
__global__ __launch_bounds__(256) void expm_params_kernel(ExpmArgs args, int32_t* params, double* norms) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (b >= args.batch) return;
  const int n = args.n;
  bool bad = false;
  double norm = 0.;
  for (int j = 0; j < P; ++j) {
    double col;
    if constexpr (P <= 8) {
      double x[P];
#pragma unroll
      for (int r = 0; r < P; ++r) {
        const bool in = r < n && j < n;
        const float a = in ? load_elem<T>(args.x, b, r, j) : 0.f;
        bad |= !finite_f32(a);
        x[r] = fabs(static_cast<double>(a));
        if constexpr (Pair) {
          const float g = in ? load_elem<T>(args.g, b, r, j) : 0.f;
          bad |= !finite_f32(g);
          x[r] += fabs(static_cast<double>(g));
        }
      }
      if constexpr (P == 4) {
        col = (x[0] + x[2]) + (x[1] + x[3]);
      } else {
        col = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
      }
    } else {
      col = 0.;
      for (int r = 0; r < P; ++r) {
        const bool in = r < n && j < n;
        const float a = in ? load_elem<T>(args.x, b, r, j) : 0.f;
        bad |= !finite_f32(a);
        col += fabs(static_cast<double>(a));
        if constexpr (Pair) {
          const float g = in ? load_elem<T>(args.g, b, r, j) : 0.f;
          bad |= !finite_f32(g);
          col += fabs(static_cast<double>(g));
        }
      }
    }
    norm = fmax(norm, col);
  }
  if (bad) {
    params[2 * b] = -1;
    params[2 * b + 1] = -1;
    if (norms) norms[b] = __builtin_nan("");
    return;
  }
  params[2 * b] = 18;  // the reference always evaluates t18 (csrc/MatrixExpSmall.cuh:163, :368)
  params[2 * b + 1] = squarings_from_norm(norm);
  if (norms) norms[b] = norm;
}

template <typename T, bool Pair>
hipError_t launch_params_t(const ExpmArgs& args, int32_t* params, double* norms, hipStream_t stream) {
  const int P = args.n <= 4 ? 4 : args.n <= 8 ? 8 : args.n <= 16 ? 16 : 32;
  const dim3 grid(static_cast<unsigned>((args.batch + 255) / 256));
  switch (P) {
    case 4: hipLaunchKernelGGL((expm_params_kernel<T, 4, Pair>), grid, dim3(256), 0, stream, args, params, norms); break;
    case 8: hipLaunchKernelGGL((expm_params_kernel<T, 8, Pair>), grid, dim3(256), 0, stream, args, params, norms); break;
    case 16: hipLaunchKernelGGL((expm_params_kernel<T, 16, Pair>), grid, dim3(256), 0, stream, args, params, norms); break;
    default: hipLaunchKernelGGL((expm_params_kernel<T, 32, Pair>), grid, dim3(256), 0, stream, args, params, norms); break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_params(const ExpmArgs& args, int dtype, bool pair, int32_t* params, double* norms,
                         hipStream_t stream) {
  if (dtype == F32::code) return pair ? launch_params_t<F32, true>(args, params, norms, stream) : launch_params_t<F32, false>(args, params, norms, stream);
  if (dtype == BF16::code) return pair ? launch_params_t<BF16, true>(args, params, norms, stream) : launch_params_t<BF16, false>(args, params, norms, stream);
  return pair ? launch_params_t<F16, true>(args, params, norms, stream) : launch_params_t<F16, false>(args, params, norms, stream);
}

}  // namespace fh

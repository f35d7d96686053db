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
// padded LDS tile (P x (P+1) floats).
//
// The MFMA pipe and the VALU do not execute concurrently on gfx950, so every
// VALU instruction adds to the MFMA time; the kernel keeps VALU work to the
// combines, one transpose per left operand and the loads/stores.  It is
// persistent: each wavefront walks matrices with a grid stride and issues the
// next matrix's loads before computing the current one.  The evaluation
// order keeps at most four powers and three temporaries live so that two
// wavefronts fit per SIMD at P = 32.
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

// B(K+1) = c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 (csrc/MatrixExpSmall.cuh:
// 268-281) with zero coefficients skipped; identity on D only.
template <int K, int P, bool Pair>
__device__ __forceinline__ PTm<P, Pair> combine(const PTm<P, Pair>& a, const PTm<P, Pair>& a2,
                                                const PTm<P, Pair>& a3, const PTm<P, Pair>& a6,
                                                const float (&diag)[TileCfg<P>::R]) {
  constexpr float c0 = kCoef[K][0], c1 = kCoef[K][1], c2 = kCoef[K][2], c3 = kCoef[K][3], c6 = kCoef[K][4];
  PTm<P, Pair> b;
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) {
    float t;
    if constexpr (c1 != 0.f) {
      t = __builtin_fmaf(c1, a.d.v[r], c0 * diag[r]);
    } else {
      t = c0 * diag[r];
    }
    t = __builtin_fmaf(c2, a2.d.v[r], t);
    t = __builtin_fmaf(c3, a3.d.v[r], t);
    if constexpr (c6 != 0.f) t = __builtin_fmaf(c6, a6.d.v[r], t);
    b.d.v[r] = t;
    if constexpr (Pair) {
      float w = (c1 != 0.f) ? __builtin_fmaf(c2, a2.u.v[r], c1 * a.u.v[r]) : c2 * a2.u.v[r];
      w = __builtin_fmaf(c3, a3.u.v[r], w);
      if constexpr (c6 != 0.f) w = __builtin_fmaf(c6, a6.u.v[r], w);
      b.u.v[r] = w;
    }
  }
  return b;
}

// Layout classes for loading: rows contiguous (sc == 1) loads the D layout of
// the matrix itself; columns contiguous (sr == 1) loads the D layout of its
// transpose; anything else gathers element-wise through the strides.
constexpr int kLoadRows = 0;
constexpr int kLoadCols = 1;

template <typename T, int P>
__device__ __forceinline__ Tm<P> load_tile(const Operand& op, int64_t b, int n, int lane, bool transposed) {
  using C = TileCfg<P>;
  const int c = C::col(lane);
  Tm<P> m;
#pragma unroll
  for (int r = 0; r < C::R; ++r) {
    const int row = C::row(lane, r);
    const bool in = row < n && c < n;
    // transposed: element (row, c) of M^T, i.e. M[c][row]
    m.v[r] = in ? load_elem_nosign<T>(op, b, transposed ? c : row, transposed ? row : c) : 0.f;
  }
  return m;
}

// Occupancy target (wavefronts per SIMD) the register allocation must meet.
template <int P, bool Pair>
constexpr int kTileWaves() {
  return P == 16 ? 4 : (Pair ? 1 : 2);
}

template <typename T, int P, bool Pair, int XL, int GL>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kTileWaves<P, Pair>(), 8))) void expm_tile_kernel(
    ExpmArgs args) {
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

  int64_t b = blockIdx.x;
  Tm<P> nx, ng;
  if (b < args.batch) {
    nx = load_tile<T, P>(args.x, b, n, lane, XL == kLoadCols);
    if constexpr (Pair) ng = load_tile<T, P>(args.g, b, n, lane, GL == kLoadCols);
  }
  for (; b < args.batch; b += gridDim.x) {
    const Tm<P> lx = nx;
    Tm<P> lg;
    if constexpr (Pair) lg = ng;
    if (b + gridDim.x < args.batch) {
      nx = load_tile<T, P>(args.x, b + gridDim.x, n, lane, XL == kLoadCols);
      if constexpr (Pair) ng = load_tile<T, P>(args.g, b + gridDim.x, n, lane, GL == kLoadCols);
    }

    // Both layouts of X (and G) through the LDS tile; the tile that holds the
    // plain layout also feeds the column sums of the norm.
    PTm<P, Pair> a, at;
    if constexpr (XL == kLoadCols) {
      at.d = lx;
      a.d = transpose<P>(lx, buf, lane);
    } else {
      a.d = lx;
      at.d = transpose<P>(lx, buf, lane);
    }
    if constexpr (Pair) {
      if constexpr (GL == kLoadCols) {
        at.u = lg;
        a.u = transpose<P>(lg, buf, lane);
      } else {
        a.u = lg;
        at.u = transpose<P>(lg, buf, lane);
      }
    }
    // FP64 1-norm, rows summed sequentially per column, |A| then |G| per row
    // (csrc/MatrixExpSmall.cuh:343-357); the total of the column sums is
    // finite exactly when every entry is (non-finite rule, :318-331).
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
    double norm = 0., total = 0.;
    for (int j = 0; j < P; ++j) {
      norm = fmax(norm, colsum[j]);
      total += colsum[j];
    }
    const bool bad = !__builtin_isfinite(total);
    const int s = bad ? 0 : squarings_from_norm(norm);
    __syncthreads();

    if (bad) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = C::row(lane, r);
        if (row < n && c < n) store_elem<T>(args.out, (b * n + row) * n + c, __builtin_nanf(""));
      }
      if (lane == 0 && args.s_out) args.s_out[b] = -1;
      continue;
    }

    // Scale by 2^-s (csrc/MatrixExpSmall.cuh:362-367), the views' lazy
    // negation folded into the same exact multiply.
    const float scale = __builtin_ldexpf(1.f, -s);
    const float scale_x = scale * args.x.sign;
    const float scale_g = scale * args.g.sign;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      a.d.v[r] *= scale_x;
      at.d.v[r] *= scale_x;
      if constexpr (Pair) {
        a.u.v[r] *= scale_g;
        at.u.v[r] *= scale_g;
      }
    }

    // Degree-18 polynomial.  Powers are formed as A.A and A.A^2 (all factors
    // are polynomials in the same matrix), then A^6 = A^3.A^3,
    // A9 = B1.B5 + B4 and T = B2 + (B3 + A9).A9.
    const PTm<P, Pair> a2 = pmm<P, Pair>(at, a);
    const PTm<P, Pair> a3 = pmm<P, Pair>(at, a2);
    const PTm<P, Pair> a6 = pmm<P, Pair>(ptranspose<P, Pair>(a3, buf, lane), a3);
    PTm<P, Pair> a9 = pmm<P, Pair>(ptranspose<P, Pair>(combine<0, P, Pair>(a, a2, a3, a6, diag), buf, lane),
                                   combine<4, P, Pair>(a, a2, a3, a6, diag));
    a9 = padd<P, Pair>(a9, combine<3, P, Pair>(a, a2, a3, a6, diag));
    const PTm<P, Pair> lhst =
        ptranspose<P, Pair>(padd<P, Pair>(combine<2, P, Pair>(a, a2, a3, a6, diag), a9), buf, lane);
    const PTm<P, Pair> b2 = combine<1, P, Pair>(a, a2, a3, a6, diag);
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

template <typename T, int P, bool Pair, int XL, int GL>
hipError_t launch_tile_l(const ExpmArgs& args, hipStream_t stream) {
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_tile_kernel<T, P, Pair, XL, GL>), 64);
  const int64_t grid = args.batch < resident ? args.batch : resident;
  hipLaunchKernelGGL((expm_tile_kernel<T, P, Pair, XL, GL>), dim3(static_cast<unsigned>(grid)), dim3(64), 0, stream,
                     args);
  return hipGetLastError();
}

int load_class(const Operand& op) { return (op.sr == 1 && op.sc != 1) ? kLoadCols : kLoadRows; }

template <typename T, int P, bool Pair>
hipError_t launch_tile_tp(const ExpmArgs& args, hipStream_t stream) {
  const int xl = load_class(args.x);
  if constexpr (Pair) {
    const int gl = load_class(args.g);
    if (xl == kLoadRows) {
      return gl == kLoadRows ? launch_tile_l<T, P, Pair, kLoadRows, kLoadRows>(args, stream)
                             : launch_tile_l<T, P, Pair, kLoadRows, kLoadCols>(args, stream);
    }
    return gl == kLoadRows ? launch_tile_l<T, P, Pair, kLoadCols, kLoadRows>(args, stream)
                           : launch_tile_l<T, P, Pair, kLoadCols, kLoadCols>(args, stream);
  } else {
    return xl == kLoadRows ? launch_tile_l<T, P, Pair, kLoadRows, kLoadRows>(args, stream)
                           : launch_tile_l<T, P, Pair, kLoadCols, kLoadRows>(args, stream);
  }
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

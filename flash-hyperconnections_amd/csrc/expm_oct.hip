// P == 8 kernel (n = 5..8) on the matrix cores: 4 matrices per 64-lane
// wavefront, every product on v_mfma_f32_4x4x1_16b_f32.  It serves the Frechet
// derivative; the forward runs the 16-matrix layout of expm_oct16.hip, which
// moves 2.5x fewer LDS bytes per product (measured: forward 8-17% faster, the
// Frechet pair there no faster -- its registers allow two wavefronts per SIMD,
// and 16 matrices square to the largest of 16 counts).
//
// Layout: an 8 x 8 matrix is a 2 x 2 arrangement of 4 x 4 blocks spread over
// one row of 16 lanes: lane l serves matrix slot m = l/16, block (I, J) with
// I = bit 3 and J = bit 2 of l, and index q = l%4 inside the block.  A
// matrix value is held in the C (column) layout of four VGPRs,
//   v[r] = M[4I + r][4J + q],
// the left operand of a product as a whole row of eight VGPRs,
//   v[k] = M[4I + q][k],  k = 0..7,
// and the right operand as a whole column of eight VGPRs,
//   v[k] = M[k][4J + q].
// The 4x4x1 MFMA multiplies 16 independent 4 x 4 blocks per instruction
// (block b's lanes supply A[i][0] from lane 4b+i and B[0][j] from lane 4b+j;
// D[i][j] lands in lane 4b+j, VGPR i), so output block (I, J) of X.Y is
//   sum over K = 0, 1 and k = 0..3 of  X_IK[:, k] (x) Y_KJ[k, :].
// Its A operand is row q of X block (I, K) and its B operand column q of Y
// block (K, J): entries 4K..4K+3 of the lane's own row and column registers,
// so no step moves data between lanes.  Steps run K = 0, 1 in turn -- the
// products accumulate k = 0..7 in the reference's order from +0, each step
// one exact FMA (csrc/MatrixExpSmall.cuh:31-33).  Rows and columns are formed
// from the C layout through the wavefront's LDS plane: one 16-byte write per
// lane, then eight 4-byte reads for a row and two 16-byte reads for a
// column.
//
// Arithmetic is the reference's, element by element (csrc/MatrixExpSmall.cuh:
// 22-106): Frechet U blocks sum D.U and U.D separately and add them, combines
// are the contracted chain with zero coefficients skipped, the FP64 norm uses
// the P = 8 butterfly.  Results are bit-identical to that evaluation up to the
// sign of zero results.
#include "fh_kernels.h"

namespace fh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kOctWaves = 4;     // wavefronts per workgroup
constexpr int kOctUnit = 4;      // matrices per wavefront
constexpr int kOctLds = 512;     // floats per wavefront: two 4 x 64 transpose planes

constexpr int kRor4 = 0x124;     // DPP row_ror:4  (lane l reads lane l - 4 of its row of 16)
constexpr int kRor8 = 0x128;     // DPP row_ror:8
constexpr int kRor12 = 0x12C;    // DPP row_ror:12 (lane l reads lane l + 4)

struct Q {
  float v[4];
};

template <bool Pair>
struct PQ {
  Q d;
  Q u;
};

// Compiler ordering of the wavefront's LDS accesses (the hardware performs
// one wavefront's LDS operations in issue order).
__device__ __forceinline__ void lds_order() {
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

// Transpose of every 4 x 4 block in place (C <-> R) through the wavefront's
// LDS plane t (256 floats): lane (b, q), b = lane/4, writes its four values
// as one 16-byte chunk to plane row q, slot b ^ 2q, and reads back element q
// of slot b from the four plane rows (XOR swizzle: no bank conflicts).
__device__ __forceinline__ void plane_write(const Q& m, float* t, int lane) {
  const int b = lane >> 2, q = lane & 3;
  *reinterpret_cast<float4*>(t + q * 64 + 4 * (b ^ (2 * q))) = make_float4(m.v[0], m.v[1], m.v[2], m.v[3]);
}
__device__ __forceinline__ Q plane_read(const float* t, int lane) {
  const int b = lane >> 2, q = lane & 3;
  Q r;
#pragma unroll
  for (int k = 0; k < 4; ++k) r.v[k] = t[k * 64 + 4 * (b ^ (2 * k)) + q];
  return r;
}

template <bool Pair>
__device__ __forceinline__ PQ<Pair> ptranspose(const PQ<Pair>& a, float* t, int lane) {
  plane_write(a.d, t, lane);
  if constexpr (Pair) plane_write(a.u, t + 256, lane);
  lds_order();
  PQ<Pair> r;
  r.d = plane_read(t, lane);
  if constexpr (Pair) r.u = plane_read(t + 256, lane);
  lds_order();
  return r;
}

// Left operands are held as whole rows: lane (m, I, J, q) keeps row 4I + q
// of its matrix, all 8 entries, so the A operand of every block step is one
// of its own registers.
struct Q8 {
  float v[8];
};
template <bool Pair>
struct PR {
  Q8 d;
  Q8 u;
};

// Row 4I + q of the matrix whose C layout sits in plane t: entries 4K..4K+3
// are row q of block (I, K), read from that block's slot as plane_read does.
__device__ __forceinline__ Q8 plane_rows(const float* t, int lane) {
  const int b = lane >> 2, q = lane & 3;
  Q8 r;
#pragma unroll
  for (int K = 0; K < 2; ++K)
#pragma unroll
    for (int k = 0; k < 4; ++k) r.v[4 * K + k] = t[k * 64 + 4 * (((b & ~1) | K) ^ (2 * k)) + q];
  return r;
}

template <bool Pair>
__device__ __forceinline__ PR<Pair> prows(const PQ<Pair>& c, float* t, int lane) {
  plane_write(c.d, t, lane);
  if constexpr (Pair) plane_write(c.u, t + 256, lane);
  lds_order();
  PR<Pair> r;
  r.d = plane_rows(t, lane);
  if constexpr (Pair) r.u = plane_rows(t + 256, lane);
  lds_order();
  return r;
}

// Whole column 4J + q of the matrix whose C layout sits in plane t: entries
// 0..3 are column q of block (0, J), entries 4..7 column q of block (1, J),
// each one 16-byte chunk of plane row q (slots as plane_write puts them).
__device__ __forceinline__ Q8 plane_cols(const float* t, int lane) {
  const int b = lane >> 2, q = lane & 3;
  const float* row = t + q * 64;
  const float4 lo = *reinterpret_cast<const float4*>(row + 4 * ((b & ~2) ^ (2 * q)));
  const float4 hi = *reinterpret_cast<const float4*>(row + 4 * ((b | 2) ^ (2 * q)));
  return Q8{{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w}};
}

template <bool Pair>
__device__ __forceinline__ PR<Pair> pcols(const PQ<Pair>& c, float* t, int lane) {
  plane_write(c.d, t, lane);
  if constexpr (Pair) plane_write(c.u, t + 256, lane);
  lds_order();
  PR<Pair> r;
  r.d = plane_cols(t, lane);
  if constexpr (Pair) r.u = plane_cols(t + 256, lane);
  lds_order();
  return r;
}

// Rows and columns of one value through a single plane write.
template <bool Pair>
__device__ __forceinline__ void prowcols(const PQ<Pair>& c, float* t, int lane, PR<Pair>& rows, PR<Pair>& cols) {
  plane_write(c.d, t, lane);
  if constexpr (Pair) plane_write(c.u, t + 256, lane);
  lds_order();
  rows.d = plane_rows(t, lane);
  cols.d = plane_cols(t, lane);
  if constexpr (Pair) {
    rows.u = plane_rows(t + 256, lane);
    cols.u = plane_cols(t + 256, lane);
  }
  lds_order();
}

// One block product chain: k = 0..7 (K = 0 block first), from +0.  Step
// (K, k) takes A = row q of X block (I, K), entry k, and B = column q of Y
// block (K, J), entry k: entries 4K + k of the lane's row and column.
__device__ __forceinline__ Q chain(const Q8& xr, const Q8& yc) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 8; ++k) acc = __builtin_amdgcn_mfma_f32_4x4x1f32(xr.v[k], yc.v[k], acc, 0, 0, 0);
  return Q{{acc[0], acc[1], acc[2], acc[3]}};
}

// Structured (Frechet) product (D1.D2, D1.U2 + U1.D2) in C layout from X as
// whole rows and Y as whole columns; the two U sums are kept separate and
// added last (csrc/MatrixExpSmall.cuh:34-49).
template <bool Pair>
__device__ __forceinline__ PQ<Pair> pmm(const PR<Pair>& xr, const PR<Pair>& yc) {
  PQ<Pair> c;
  c.d = chain(xr.d, yc.d);
  if constexpr (Pair) {
    const Q u = chain(xr.d, yc.u);
    const Q v = chain(xr.u, yc.d);
#pragma unroll
    for (int r = 0; r < 4; ++r) c.u.v[r] = u.v[r] + v.v[r];
  }
  return c;
}

// B(K+1) = c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 in C layout, the contracted
// chain of csrc/MatrixExpSmall.cuh:74-77 with zero coefficients skipped;
// `diag` is 1 in the VGPR holding a diagonal entry and 0 elsewhere.  U blocks
// have no identity term and start from c1*A.
template <int K, bool Pair>
__device__ __forceinline__ PQ<Pair> comb(const PQ<Pair>& a, const PQ<Pair>& a2, const PQ<Pair>& a3,
                                         const PQ<Pair>& a6, const Q& diag) {
  constexpr float c0 = kCoef[K][0], c1 = kCoef[K][1], c2 = kCoef[K][2], c3 = kCoef[K][3], c6 = kCoef[K][4];
  PQ<Pair> b;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    // c0 * I, with +0 from a VGPR where c0 is 0 (see vgpr_zero).
    const float i0 = c0 != 0.f ? c0 * diag.v[r] : vgpr_zero();
    float t;
    if constexpr (c1 != 0.f) {
      t = __builtin_fmaf(c1, a.d.v[r], i0);
      t = __builtin_fmaf(c2, a2.d.v[r], t);
    } else {
      t = __builtin_fmaf(c2, a2.d.v[r], i0);
    }
    t = __builtin_fmaf(c3, a3.d.v[r], t);
    if constexpr (c6 != 0.f) t = __builtin_fmaf(c6, a6.d.v[r], t);
    b.d.v[r] = t;
    if constexpr (Pair) {
      float w;
      if constexpr (c1 != 0.f) {
        w = c1 * a.u.v[r];
        w = __builtin_fmaf(c2, a2.u.v[r], w);
      } else {
        w = c2 * a2.u.v[r];
      }
      w = __builtin_fmaf(c3, a3.u.v[r], w);
      if constexpr (c6 != 0.f) w = __builtin_fmaf(c6, a6.u.v[r], w);
      b.u.v[r] = w;
    }
  }
  return b;
}

template <bool Pair>
__device__ __forceinline__ PQ<Pair> padd(const PQ<Pair>& a, const PQ<Pair>& b) {
  PQ<Pair> c;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    c.d.v[r] = a.d.v[r] + b.d.v[r];
    if constexpr (Pair) c.u.v[r] = a.u.v[r] + b.u.v[r];
  }
  return c;
}

// Degree-18 polynomial of the scaled pair in both layouts
// (csrc/MatrixExpSmall.cuh:83-106): A2 = A.A, A3 = A2.A, A6 = A3.A3,
// A9 = B1.B5 + B4, T = B2 + (B3 + A9).A9.  Result in C layout.
template <bool Pair>
__device__ __forceinline__ PQ<Pair> t18(const PR<Pair>& ar, const PR<Pair>& acol, const PQ<Pair>& ac,
                                        const Q& diag, float* t, int lane) {
  const PQ<Pair> a2 = pmm<Pair>(ar, acol);
  const PQ<Pair> a3 = pmm<Pair>(prows<Pair>(a2, t, lane), acol);
  PR<Pair> a3r, a3c;
  prowcols<Pair>(a3, t, lane, a3r, a3c);
  const PQ<Pair> a6 = pmm<Pair>(a3r, a3c);
  const PR<Pair> b1r = prows<Pair>(comb<0, Pair>(ac, a2, a3, a6, diag), t, lane);
  PQ<Pair> a9 = pmm<Pair>(b1r, pcols<Pair>(comb<4, Pair>(ac, a2, a3, a6, diag), t, lane));
  a9 = padd<Pair>(a9, comb<3, Pair>(ac, a2, a3, a6, diag));
  const PR<Pair> lhsr = prows<Pair>(padd<Pair>(comb<2, Pair>(ac, a2, a3, a6, diag), a9), t, lane);
  return padd<Pair>(comb<1, Pair>(ac, a2, a3, a6, diag), pmm<Pair>(lhsr, pcols<Pair>(a9, t, lane)));
}

// ---- norm ---------------------------------------------------------------------

// Exchange with the lane whose bank index differs in bit 0 (lane ^ 4) or bit 1
// (lane ^ 8) within the row of 16.
__device__ __forceinline__ int xor4_i(int v) {
  const int t = __builtin_amdgcn_update_dpp(v, v, kRor4, 0xF, 0xA, false);
  return __builtin_amdgcn_update_dpp(t, v, kRor12, 0xF, 0x5, false);
}
__device__ __forceinline__ int xor8_i(int v) { return __builtin_amdgcn_update_dpp(v, v, kRor8, 0xF, 0xF, false); }
__device__ __forceinline__ double xor8_d(double v) {
  const int2 w = __builtin_bit_cast(int2, v);
  return __builtin_bit_cast(double, make_int2(xor8_i(w.x), xor8_i(w.y)));
}
template <int Ctrl>
__device__ __forceinline__ double dpp_d(double v) {
  const int2 w = __builtin_bit_cast(int2, v);
  return __builtin_bit_cast(double, make_int2(__builtin_amdgcn_update_dpp(w.x, w.x, Ctrl, 0xF, 0xF, false),
                                              __builtin_amdgcn_update_dpp(w.y, w.y, Ctrl, 0xF, 0xF, false)));
}
__device__ __forceinline__ double xor4_d(double v) {
  const int2 w = __builtin_bit_cast(int2, v);
  return __builtin_bit_cast(double, make_int2(xor4_i(w.x), xor4_i(w.y)));
}

// Maximum of a non-negative float's bit pattern over the 8 columns of the
// lane's matrix (lanes differing in bits 0, 1 and the bank's J bit).
__device__ __forceinline__ uint32_t matrix_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0xB1, 0xF, 0xF, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), 0x4E, 0xF, 0xF, false)));
  return max(v, static_cast<uint32_t>(xor4_i(static_cast<int>(v))));
}

// Squaring count of the lane's matrix, or -1 for a non-finite one.  The FP32
// estimate of the column-sum norm decides s unless it lies near a squaring
// boundary (squarings_from_estimate); then the matrix takes the reference's
// FP64 norm: per column the butterfly ((x0 + x4) + (x2 + x6)) +
// ((x1 + x5) + (x3 + x7)) with x_r = |A[r][j]| (+ |G[r][j]|)
// (csrc/MatrixExpSmall.cuh:144-152), whose total is finite exactly when every
// entry is (:126-140).  The lanes of blocks (0, J) and (1, J) hold rows 0-3
// and 4-7 of the same columns.
template <bool Pair>
__device__ __forceinline__ int matrix_squarings(const PQ<Pair>& ac, int I) {
  float p = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p += __builtin_fabsf(ac.d.v[r]);
    if constexpr (Pair) p += __builtin_fabsf(ac.u.v[r]);
  }
  p += __int_as_float(xor8_i(__float_as_int(p)));
  const uint32_t top = matrix_max_u32(__float_as_uint(p) & 0x7FFFFFFFu);
  int s;
  const bool decided = squarings_from_estimate(__uint_as_float(top), s);
  if (__builtin_amdgcn_ballot_w64(!decided) == 0) return s;
  // Some matrix needs the exact norm: the whole wavefront computes it (the DPP
  // exchanges need every lane) and the decided matrices keep their estimate.
  double own[4], other[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    own[r] = fabs(static_cast<double>(ac.d.v[r]));
    if constexpr (Pair) own[r] += fabs(static_cast<double>(ac.u.v[r]));
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) other[r] = xor8_d(own[r]);
  double x[8];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    x[r] = I == 0 ? own[r] : other[r];
    x[4 + r] = I == 0 ? other[r] : own[r];
  }
  double norm = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
  double total = norm;
  norm = fmax(norm, dpp_d<0xB1>(norm));
  total = total + dpp_d<0xB1>(total);
  norm = fmax(norm, dpp_d<0x4E>(norm));
  total = total + dpp_d<0x4E>(total);
  norm = fmax(norm, xor4_d(norm));
  total = total + xor4_d(total);
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
struct Raw4 {
  typename T::storage v[4];
};

template <typename T, int L>
__device__ __forceinline__ Raw4<T> load_raw(const Operand& op, int64_t m, int I, int J, int q, int n, bool valid) {
  using S = typename T::storage;
  Raw4<T> w;
#pragma unroll
  for (int r = 0; r < 4; ++r) w.v[r] = S{};
  if (!valid) return w;
  const S* base = static_cast<const S*>(op.data) + m * op.sb;
  if constexpr (L == kVecRows) {
    typedef S S4 __attribute__((ext_vector_type(4)));
    const S4 x = *reinterpret_cast<const S4*>(base + (4 * I + q) * op.sr + 4 * J);
#pragma unroll
    for (int r = 0; r < 4; ++r) w.v[r] = x[r];
  } else if constexpr (L == kVecCols) {
    typedef S S4 __attribute__((ext_vector_type(4)));
    const S4 x = *reinterpret_cast<const S4*>(base + (4 * J + q) * op.sc + 4 * I);
#pragma unroll
    for (int r = 0; r < 4; ++r) w.v[r] = x[r];
  } else {
    const int col = 4 * J + q;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * I + r;
      if (row < n && col < n) w.v[r] = base[row * op.sr + col * op.sc];
    }
  }
  return w;
}

template <typename T>
__device__ __forceinline__ Q to_q(const Raw4<T>& w) {
  Q m;
#pragma unroll
  for (int r = 0; r < 4; ++r) m.v[r] = to_f32<T>(w.v[r]);
  return m;
}

template <typename T, bool Pair, int XL, int GL>
struct UnitRaw {
  Raw4<T> x;
  Raw4<T> g;
};

// ---- kernel -----------------------------------------------------------------

// Each wavefront walks 4-matrix units with a grid stride, loading a unit at
// its start (no prefetch of the next; the grid holds four times the resident
// workgroups, so the hardware starts a workgroup as another retires).  Four
// wavefronts per SIMD (at most 128 VGPRs).
template <typename T, bool Pair, int XL, int GL>
__global__ __launch_bounds__(64 * kOctWaves) __attribute__((amdgpu_waves_per_eu(4, 8))) void expm_oct_kernel(ExpmArgs args) {
  using S = typename T::storage;
  __shared__ float lds[kOctWaves][kOctLds];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float* t = lds[wave];
  const int slot = lane >> 4;
  const int I = (lane >> 3) & 1;
  const int J = (lane >> 2) & 1;
  const int q = lane & 3;
  const int n = (XL != kVecNone) ? 8 : args.n;
  Q diag;
#pragma unroll
  for (int r = 0; r < 4; ++r) diag.v[r] = (I == J && r == q) ? 1.f : 0.f;
  const int64_t units = (args.batch + kOctUnit - 1) / kOctUnit;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kOctWaves;
  int64_t unit = static_cast<int64_t>(blockIdx.x) * kOctWaves + wave;

  auto load_unit = [&](int64_t u) {
    UnitRaw<T, Pair, XL, GL> r;
    const int64_t m = u * kOctUnit + slot;
    const bool valid = m < args.batch;
    r.x = load_raw<T, XL>(args.x, m, I, J, q, n, valid);
    if constexpr (Pair) r.g = load_raw<T, GL>(args.g, m, I, J, q, n, valid);
    return r;
  };

  for (; unit < units; unit += stride) {
    const int64_t m = unit * kOctUnit + slot;
    const bool valid = m < args.batch;
    const UnitRaw<T, Pair, XL, GL> raw = load_unit(unit);
    PQ<Pair> lx;  // as loaded: R layout for kVecRows, C layout otherwise
    lx.d = to_q<T>(raw.x);
    if constexpr (Pair) lx.u = to_q<T>(raw.g);

    // X (and G) in the C layout and as whole rows.
    PQ<Pair> ac;
    if constexpr (XL == kVecRows || GL == kVecRows) {
      const PQ<Pair> other = ptranspose<Pair>(lx, t, lane);
      ac.d = XL == kVecRows ? other.d : lx.d;
      if constexpr (Pair) ac.u = GL == kVecRows ? other.u : lx.u;
    } else {
      ac = lx;
    }
    const int s = matrix_squarings<Pair>(ac, I);
    const bool bad = s < 0;

    // Scale by 2^-s (csrc/MatrixExpSmall.cuh:157-162) with the views' lazy
    // negation folded into the same exact multiply, before the rows and
    // columns are formed: the LDS moves copy the scaled values as they are,
    // so one multiply per C-layout entry serves all three layouts.
    const float scale = __builtin_ldexpf(1.f, bad ? 0 : -s);
    const float scale_x = scale * args.x.sign;
    const float scale_g = scale * args.g.sign;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ac.d.v[r] *= scale_x;
      if constexpr (Pair) ac.u.v[r] *= scale_g;
    }
    PR<Pair> ar, acol;
    prowcols<Pair>(ac, t, lane, ar, acol);

    PQ<Pair> res = t18<Pair>(ar, acol, ac, diag, t, lane);

    // s squarings per matrix (csrc/MatrixExpSmall.cuh:168); the wavefront
    // loops while any of its matrices still needs one and each keeps its own
    // result.
    for (int it = 0; __builtin_amdgcn_ballot_w64(it < s) != 0; ++it) {
      PR<Pair> rr, rc;
      prowcols<Pair>(res, t, lane, rr, rc);
      PQ<Pair> sq;
      if constexpr (Pair) {
        if (__builtin_amdgcn_ballot_w64(it + 1 < s) == 0) {
          // The wavefront's last round: nothing reads its D block, so only
          // the U sums run (as pmm forms them).
          const Q u = chain(rr.d, rc.u);
          const Q v = chain(rr.u, rc.d);
#pragma unroll
          for (int r = 0; r < 4; ++r) sq.u.v[r] = u.v[r] + v.v[r];
          sq.d = res.d;
        } else {
          sq = pmm<Pair>(rr, rc);
        }
      } else {
        sq = pmm<Pair>(rr, rc);
      }
      const bool keep = it < s;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        res.d.v[r] = keep ? sq.d.v[r] : res.d.v[r];
        if constexpr (Pair) res.u.v[r] = keep ? sq.u.v[r] : res.u.v[r];
      }
    }

    Q out = Pair ? res.u : res.d;
    if (bad) {
#pragma unroll
      for (int r = 0; r < 4; ++r) out.v[r] = __builtin_nanf("");
    }
    if constexpr (XL != kVecNone) {
      // n == 8: each lane writes 4 consecutive entries of a row from the R layout.
      plane_write(out, t, lane);
      lds_order();
      const Q row = plane_read(t, lane);
      lds_order();
      if (valid) {
        typedef S S4 __attribute__((ext_vector_type(4)));
        S4 w;
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = from_f32<T>(row.v[k]);
        __builtin_nontemporal_store(w, reinterpret_cast<S4*>(static_cast<S*>(args.out) + m * 64 + (4 * I + q) * 8 + 4 * J));
      }
    } else if (valid) {
      S* o = static_cast<S*>(args.out) + m * n * n;
      const int col = 4 * J + q;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * I + r;
        if (row < n && col < n) __builtin_nontemporal_store(from_f32<T>(out.v[r]), &o[row * n + col]);
      }
    }
    if (valid && (lane & 15) == 0 && args.s_out) args.s_out[m] = s;
  }
}

template <typename T, bool Pair, int XL, int GL>
hipError_t launch_oct_l(const ExpmArgs& args, hipStream_t stream) {
  // Four times the resident workgroups: against one unit per wavefront the
  // p8 Frechet kernel ran 116.0 -> 113.2 and 116.8 -> 112.7 us (same process,
  // alternating; 8x resident in between).
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_oct_kernel<T, Pair, XL, GL>), 64 * kOctWaves);
  const int64_t units = (args.batch + kOctUnit - 1) / kOctUnit;
  int64_t grid = (units + kOctWaves - 1) / kOctWaves;
  if (grid > 4 * resident) grid = 4 * resident;
  hipLaunchKernelGGL((expm_oct_kernel<T, Pair, XL, GL>), dim3(static_cast<unsigned>(grid)), dim3(64 * kOctWaves), 0,
                     stream, args);
  return hipGetLastError();
}

// n < 8 or an unclassified stride pattern takes the element-wise loader; for
// n == 8 each operand is classified independently (the output is row-major).
template <typename T, bool Pair>
hipError_t launch_oct_t(const ExpmArgs& args, hipStream_t stream) {
  const int xl = args.n == 8 ? args.x.vec : kVecNone;
  const int gl = (Pair && args.n == 8) ? args.g.vec : kVecNone;
  if (xl == kVecNone || (Pair && gl == kVecNone)) return launch_oct_l<T, Pair, kVecNone, kVecNone>(args, stream);
  if constexpr (Pair) {
    if (xl == kVecRows) {
      return gl == kVecRows ? launch_oct_l<T, Pair, kVecRows, kVecRows>(args, stream)
                            : launch_oct_l<T, Pair, kVecRows, kVecCols>(args, stream);
    }
    return gl == kVecRows ? launch_oct_l<T, Pair, kVecCols, kVecRows>(args, stream)
                          : launch_oct_l<T, Pair, kVecCols, kVecCols>(args, stream);
  } else {
    return xl == kVecRows ? launch_oct_l<T, Pair, kVecRows, kVecNone>(args, stream)
                          : launch_oct_l<T, Pair, kVecCols, kVecNone>(args, stream);
  }
}

}  // namespace

hipError_t launch_oct(const ExpmArgs& args, int dtype, bool pair, hipStream_t stream) {
  if (!pair) return launch_oct16(args, dtype, stream);
  if (dtype == F32::code) return launch_oct_t<F32, true>(args, stream);
  if (dtype == BF16::code) return launch_oct_t<BF16, true>(args, stream);
  return launch_oct_t<F16, true>(args, stream);
}

}  // namespace fh

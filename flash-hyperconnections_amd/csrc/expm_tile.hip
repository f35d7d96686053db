// P in {16, 32} kernel (n = 9..32): one 64-lane wavefront per matrix, every
// product on FP32 MFMA (v_mfma_f32_16x16x4_f32 for P = 16,
// v_mfma_f32_32x32x2_f32 for P = 32).
//
// Layout: a P x P matrix occupies R = P*P/64 VGPRs per lane in the MFMA
// accumulator ("D") layout: lane l, VGPR r holds M[row(l, r)][l % P] with
//   P = 16: row = 4*(l/16) + r
//   P = 32: row = 8*(r/4) + 4*(l/32) + r%4,
// i.e. row(l, r) = row0(l) + step(r).  Step r of a product feeds the A
// operand from VGPR r of X^T and the B operand from VGPR r of Y; lane group g
// then contributes k = row(g, r), so the R steps together cover k = 0..P-1 and
//   X.Y = sum_r mfma(a = (X^T).v[r], b = Y.v[r])
// needs no data movement for Y.  Left operands are transposed through a
// padded LDS tile (P x (P+1) floats); the workgroup is the one wavefront,
// whose LDS accesses complete in issue order, so the transposes need
// compiler ordering only, no barrier and no wait.
//
// On gfx950 the MFMA pipe and the VALU barely overlap (about 15% when
// different wavefronts of a SIMD feed them; not at all within one), so every
// VALU instruction adds to the MFMA time.  The kernel therefore keeps VALU
// work to the combines:
// * loads and stores go through buffer resources: one per-lane offset fixed
//   for the whole kernel, the per-VGPR row offsets in scalar registers and
//   the matrix base in the descriptor, so addressing costs no VALU;
// * no prefetch of a next matrix, on a grid of one wavefront per matrix
//   (P = 32) or four times the resident workgroups (P = 16): against a
//   persistent grid that prefetched the next matrix's storage bits, the
//   forward at config 5 ran 151.3 -> 143.7 us, and without the prefetch's
//   registers no Frechet variant spills and the P = 16 one runs six
//   wavefronts per SIMD instead of five;
// * s comes from an FP32 estimate of the norm (a few adds and a cross-lane
//   maximum) whenever that estimate decides it exactly; the FP64 sequential
//   column sums of the reference run only near a squaring boundary or for
//   non-finite input;
// * the Frechet half D1.U2 + U1.D2 is one accumulation chain, fed step by
//   step together with the D chain (two independent MFMA chains, and each
//   operand register dies after its step).
// Each FP32 MFMA step equals an fmaf chain over its k terms in ascending
// order, so results differ from the reference's sequential FMA chains only
// through the order of the k terms within a product and that one U chain
// (parity is by tolerance; s is bit-identical).
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
  __device__ static constexpr int step(int r) { return r; }
  __device__ static __forceinline__ int row0(int lane) { return 4 * (lane >> 4); }
  __device__ static __forceinline__ int col(int lane) { return lane & 15; }
  // VGPR holding this lane's diagonal entry, -1 when it holds none.
  __device__ static __forceinline__ int diag_reg(int lane) { return (lane >> 4) == ((lane & 15) >> 2) ? (lane & 3) : -1; }
  __device__ static __forceinline__ acc_t mfma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

template <>
struct TileCfg<32> {
  static constexpr int R = 16;
  using acc_t = v16f;
  __device__ static constexpr int step(int r) { return 8 * (r >> 2) + (r & 3); }
  __device__ static __forceinline__ int row0(int lane) { return 4 * (lane >> 5); }
  __device__ static __forceinline__ int col(int lane) { return lane & 31; }
  __device__ static __forceinline__ int diag_reg(int lane) {
    const int c = lane & 31;
    return ((c >> 2) & 1) == (lane >> 5) ? 4 * (c >> 3) + (c & 3) : -1;
  }
  __device__ static __forceinline__ acc_t mfma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

template <int P>
using Acc = typename TileCfg<P>::acc_t;

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
__device__ __forceinline__ Acc<P> to_acc(const Tm<P>& m) {
  Acc<P> a;
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) a[r] = m.v[r];
  return a;
}
template <int P>
__device__ __forceinline__ Tm<P> from_acc(const Acc<P>& a) {
  Tm<P> m;
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) m.v[r] = a[r];
  return m;
}

// acc + X.Y, X given as X^T in the D layout.
template <int P>
__device__ __forceinline__ Acc<P> mma(const Tm<P>& xt, const Tm<P>& y, Acc<P> acc) {
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) acc = TileCfg<P>::mfma(xt.v[r], y.v[r], acc);
  return acc;
}

// (D1, U1).(D2, U2) = (D1.D2, D1.U2 + U1.D2).  Step r feeds all three
// products, so each operand register dies after its step and the D and U
// accumulations alternate as two independent MFMA chains.  WantD = false
// skips the D chain (a last squaring, whose D block nothing reads); the D
// block is then left as x's.
template <int P, bool Pair, bool WantD = true>
__device__ __forceinline__ PTm<P, Pair> pmm(const PTm<P, Pair>& xt, const PTm<P, Pair>& y) {
  Acc<P> d = {}, u = {};
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) {
    if constexpr (WantD) d = TileCfg<P>::mfma(xt.d.v[r], y.d.v[r], d);
    if constexpr (Pair) {
      u = TileCfg<P>::mfma(xt.d.v[r], y.u.v[r], u);
      u = TileCfg<P>::mfma(xt.u.v[r], y.d.v[r], u);
    }
  }
  PTm<P, Pair> out;
  if constexpr (WantD) {
    out.d = from_acc<P>(d);
  } else {
    out.d = y.d;
  }
  if constexpr (Pair) out.u = from_acc<P>(u);
  return out;
}

// Compiler ordering of the wavefront's LDS accesses (the hardware already
// performs one wavefront's LDS operations in issue order).
__device__ __forceinline__ void lds_order() {
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

template <int P>
__device__ __forceinline__ void tile_write(const Tm<P>& m, float* buf, int lane) {
  using C = TileCfg<P>;
  constexpr int LD = P + 1;
  const int c = C::col(lane);
  const int r0 = C::row0(lane);
#pragma unroll
  for (int r = 0; r < C::R; ++r) buf[(r0 + C::step(r)) * LD + c] = m.v[r];
}
template <int P>
__device__ __forceinline__ Tm<P> tile_read_transposed(const float* buf, int lane) {
  using C = TileCfg<P>;
  constexpr int LD = P + 1;
  const int c = C::col(lane);
  const int r0 = C::row0(lane);
  Tm<P> t;
#pragma unroll
  for (int r = 0; r < C::R; ++r) t.v[r] = buf[c * LD + r0 + C::step(r)];
  return t;
}

// D layout of M -> D layout of M^T (both halves of a pair in one round).
template <int P, bool Pair>
__device__ __forceinline__ PTm<P, Pair> ptranspose(const PTm<P, Pair>& a, float* buf, int lane) {
  constexpr int T = P * (P + 1);
  tile_write<P>(a.d, buf, lane);
  if constexpr (Pair) tile_write<P>(a.u, buf + T, lane);
  lds_order();
  PTm<P, Pair> t;
  t.d = tile_read_transposed<P>(buf, lane);
  if constexpr (Pair) t.u = tile_read_transposed<P>(buf + T, lane);
  lds_order();
  return t;
}

// c0*I in the D layout for the two combines with an identity term (B3 and B4,
// reference csrc/MatrixExpSmall.cuh:268-281), from `dreg`, the VGPR of this
// lane's diagonal entry (-1 for none).  P = 16 keeps the 2R values in
// registers for the whole kernel (it has registers to spare); P = 32 selects
// them where they are used.
template <int P>
struct Ident {
  int dreg;
  __device__ __forceinline__ float value(int k, int r) const { return dreg == r ? kCoef[k][0] : 0.f; }
};
template <>
struct Ident<16> {
  Tm<16> b3, b4;
  __device__ __forceinline__ float value(int k, int r) const { return k == 2 ? b3.v[r] : b4.v[r]; }
};
template <int P>
__device__ __forceinline__ Ident<P> make_ident(int dreg) {
  Ident<P> id;
  if constexpr (P == 16) {
#pragma unroll
    for (int r = 0; r < TileCfg<P>::R; ++r) {
      id.b3.v[r] = dreg == r ? kCoef[2][0] : 0.f;
      id.b4.v[r] = dreg == r ? kCoef[3][0] : 0.f;
    }
  } else {
    id.dreg = dreg;
  }
  return id;
}

// B(K+1) = c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 (reference
// csrc/MatrixExpSmall.cuh:268-281), the contracted chain with zero
// coefficients skipped; the identity term (D only) comes from `id`.
template <int K, int P, bool Pair>
__device__ __forceinline__ PTm<P, Pair> combine(const PTm<P, Pair>& a, const PTm<P, Pair>& a2,
                                                const PTm<P, Pair>& a3, const PTm<P, Pair>& a6, const Ident<P>& id) {
  using C = TileCfg<P>;
  constexpr float c0 = kCoef[K][0], c1 = kCoef[K][1], c2 = kCoef[K][2], c3 = kCoef[K][3], c6 = kCoef[K][4];
  static_assert(c0 == 0.f || K == 2 || K == 3, "identity terms are B3 and B4");
  PTm<P, Pair> b;
#pragma unroll
  for (int r = 0; r < C::R; ++r) {
    float t = 0.f;
    if constexpr (c0 != 0.f) t = id.value(K, r);
    if constexpr (c1 != 0.f) t = __builtin_fmaf(c1, a.d.v[r], t);
    t = __builtin_fmaf(c2, a2.d.v[r], t);
    t = __builtin_fmaf(c3, a3.d.v[r], t);
    if constexpr (c6 != 0.f) t = __builtin_fmaf(c6, a6.d.v[r], t);
    b.d.v[r] = t;
    if constexpr (Pair) {
      float w = 0.f;
      if constexpr (c1 != 0.f) w = __builtin_fmaf(c1, a.u.v[r], w);
      w = __builtin_fmaf(c2, a2.u.v[r], w);
      w = __builtin_fmaf(c3, a3.u.v[r], w);
      if constexpr (c6 != 0.f) w = __builtin_fmaf(c6, a6.u.v[r], w);
      b.u.v[r] = w;
    }
  }
  return b;
}

template <int P, bool Pair>
__device__ __forceinline__ PTm<P, Pair> padd(const PTm<P, Pair>& x, const PTm<P, Pair>& y) {
  PTm<P, Pair> z;
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) {
    z.d.v[r] = x.d.v[r] + y.d.v[r];
    if constexpr (Pair) z.u.v[r] = x.u.v[r] + y.u.v[r];
  }
  return z;
}

// Layout classes for loading: rows contiguous (kLoadRows) loads the D layout
// of the matrix itself; columns contiguous (kLoadCols) loads the D layout of
// its transpose.  Either works for any strides; the class only decides which
// of the two layouts comes from memory and which from the LDS transpose.
constexpr int kLoadRows = 0;
constexpr int kLoadCols = 1;

// Byte addressing of one operand in the D layout of the loaded matrix: the
// matrix base goes into the descriptor, `lane_off` is this lane's offset for
// VGPR 0 and step(r) * `major` the uniform offset of VGPR r.
struct TileSrc {
  const char* data;
  int64_t sb;        // bytes per batch step
  int32_t major;     // bytes per D-layout row step
  int32_t lane_off;  // bytes, VGPR 0 of this lane
  uint32_t records;  // footprint of one matrix in bytes
};

template <typename T, int P>
__device__ __forceinline__ TileSrc make_src(const Operand& op, int layout, int n, int lane) {
  using C = TileCfg<P>;
  constexpr int es = ElemIO<T>::bytes;
  const int64_t major = layout == kLoadCols ? op.sc : op.sr;
  const int64_t minor = layout == kLoadCols ? op.sr : op.sc;
  TileSrc s;
  s.data = static_cast<const char*>(op.data);
  s.sb = op.sb * es;
  s.major = static_cast<int32_t>(major * es);
  s.lane_off = static_cast<int32_t>((C::row0(lane) * major + C::col(lane) * minor) * es);
  s.records = static_cast<uint32_t>(((n - 1) * (op.sr + op.sc) + 1) * es);
  return s;
}

template <typename T, int P>
struct RawTile {
  typename ElemIO<T>::raw_t v[TileCfg<P>::R];
};

// Storage bits of matrix b; entries outside the n x n block read as +0.
template <typename T, int P, bool Full>
__device__ __forceinline__ RawTile<T, P> load_raw(const TileSrc& s, int64_t b, int n, int lane) {
  using C = TileCfg<P>;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(s.data + b * s.sb, s.records);
  RawTile<T, P> t;
  if constexpr (Full) {
#pragma unroll
    for (int r = 0; r < C::R; ++r) t.v[r] = ElemIO<T>::load(rs, s.lane_off, C::step(r) * s.major);
  } else {
    const bool col_ok = C::col(lane) < n;
#pragma unroll
    for (int r = 0; r < C::R; ++r) {
      const bool ok = col_ok && C::row0(lane) + C::step(r) < n;
      t.v[r] = ElemIO<T>::load(rs, ok ? s.lane_off + C::step(r) * s.major : kOutOfRange, 0);
    }
  }
  return t;
}

template <typename T, int P>
__device__ __forceinline__ Tm<P> to_tile(const RawTile<T, P>& raw) {
  Tm<P> m;
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) m.v[r] = ElemIO<T>::value(raw.v[r]);
  return m;
}

// Contiguous [batch, n, n] output in the input dtype.
template <typename T, int P, bool Full>
__device__ __forceinline__ void store_tile(void* out, int64_t b, int n, int lane, const Tm<P>& m) {
  using C = TileCfg<P>;
  constexpr int es = ElemIO<T>::bytes;
  const int64_t nn = static_cast<int64_t>(n) * n;
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(static_cast<char*>(out) + b * nn * es, static_cast<uint32_t>(nn * es));
  const int32_t lane_off = (C::row0(lane) * n + C::col(lane)) * es;
  if constexpr (Full) {
#pragma unroll
    for (int r = 0; r < C::R; ++r) ElemIO<T>::template store<kNontemporal>(m.v[r], rs, lane_off + C::step(r) * P * es, 0);
  } else {
    const bool col_ok = C::col(lane) < n;
#pragma unroll
    for (int r = 0; r < C::R; ++r) {
      const bool ok = col_ok && C::row0(lane) + C::step(r) < n;
      ElemIO<T>::template store<kNontemporal>(m.v[r], rs, ok ? lane_off + C::step(r) * n * es : kOutOfRange, 0);
    }
  }
}

// Maximum over the lanes of a row of 16 (every lane of the row gets it).
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xF, 0xF, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x140, 0xF, 0xF, false)));
  return v;
}

// FP32 estimate of the 1-norm max_j sum_i |A[i][j]| (+ |G[i][j]|) from the D
// layout of A (and G): each lane sums its column entries, the lanes sharing a
// column add up, and the column maximum is taken on the bit patterns (equal
// order for non-negative floats; NaN and inf compare above every finite
// value).  Relative error at most (2R + 2) * 2^-24 < 2^-18.
template <int P, bool Pair>
__device__ __forceinline__ float norm_estimate(const PTm<P, Pair>& a) {
  float p = 0.f;
#pragma unroll
  for (int r = 0; r < TileCfg<P>::R; ++r) {
    p += __builtin_fabsf(a.d.v[r]);
    if constexpr (Pair) p += __builtin_fabsf(a.u.v[r]);
  }
  if constexpr (P == 16) p += __shfl_xor(p, 16);
  p += __shfl_xor(p, 32);
  uint32_t m = row_max_u32(__float_as_uint(p) & 0x7FFFFFFFu);
  uint32_t top = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), 0));
  if constexpr (P == 32) top = max(top, static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), 16)));
  return __uint_as_float(top);
}

// The reference's FP64 norm (csrc/MatrixExpSmall.cuh:343-357): per column the
// rows summed sequentially, |A| then |G| per row, then the column maximum; the
// total of the column sums is finite exactly when every entry is (non-finite
// rule, :318-331), i.e. when every column sum is.  Returns false for
// non-finite input.  This path is rare, so it is written for few live
// registers: the row loop is not unrolled, and the maximum over columns reads
// each lane's sum into scalar registers (the order of a maximum is free).
template <int P, bool Pair>
__device__ __forceinline__ bool exact_squarings(const PTm<P, Pair>& a, float* buf, int lane, int& s) {
  constexpr int LD = P + 1;
  tile_write<P>(a.d, buf, lane);
  if constexpr (Pair) tile_write<P>(a.u, buf + P * LD, lane);
  lds_order();
  double v = 0.;
  if (lane < P) {
#pragma unroll 1
    for (int row = 0; row < P; ++row) {
      v += fabs(static_cast<double>(buf[row * LD + lane]));
      if constexpr (Pair) v += fabs(static_cast<double>(buf[P * LD + row * LD + lane]));
    }
  }
  lds_order();
  if (__builtin_amdgcn_ballot_w64(!__builtin_isfinite(v)) != 0) return false;
  double norm = 0.;
  const uint64_t bits = __builtin_bit_cast(uint64_t, v);
  const int vlo = static_cast<int>(bits), vhi = static_cast<int>(bits >> 32);
#pragma unroll 1
  for (int j = 0; j < P; ++j) {
    const uint64_t w = static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(vlo, j))) |
                       (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(vhi, j))) << 32);
    norm = fmax(norm, __builtin_bit_cast(double, w));
  }
  s = squarings_from_norm(norm);
  return true;
}

// Occupancy target (wavefronts per SIMD) the register allocation must meet.
template <int P, bool Pair>
constexpr int kTileWaves() {
  return P == 16 ? 4 : (Pair ? 2 : 3);
}

template <typename T, int P, bool Pair, int XL, int GL, bool Full>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kTileWaves<P, Pair>(), 8))) void expm_tile_kernel(
    ExpmArgs args) {
  using C = TileCfg<P>;
  constexpr int R = C::R;
  __shared__ float buf[2 * P * (P + 1)];
  const int lane = threadIdx.x;
  const int n = Full ? P : args.n;
  const TileSrc sx = make_src<T, P>(args.x, XL, n, lane);
  const TileSrc sg = make_src<T, P>(args.g, GL, n, lane);

  int64_t b = blockIdx.x;
  const int dreg_lane = C::diag_reg(lane);
  Ident<P> id_lane;
  if constexpr (P == 16) {
    id_lane = make_ident<P>(dreg_lane);
#pragma unroll
    for (int r = 0; r < R; ++r) asm volatile("" : "+v"(id_lane.b3.v[r]), "+v"(id_lane.b4.v[r]));
  }
  for (; b < args.batch; b += gridDim.x) {
    // For P = 32, opaque per matrix so that the identity terms are selected
    // where they are used instead of being kept live across the loop.
    Ident<P> id;
    if constexpr (P == 16) {
      id = id_lane;
    } else {
      int dreg = dreg_lane;
      asm volatile("" : "+v"(dreg));
      id = make_ident<P>(dreg);
    }
    // n < P = 32: the per-VGPR bounds predicates and offsets are formed
    // afresh for each matrix from an opaque copy of the lane's offsets, so
    // that they are not kept live across the loop (2R-3R registers these
    // kernels do not have; P = 16 keeps them).
    TileSrc sxm = sx, sgm = sg;
    int lane_m = lane;
    if constexpr (!Full && P == 32) {
      asm volatile("" : "+v"(sxm.lane_off), "+v"(sgm.lane_off), "+v"(lane_m));
    }
    const Tm<P> lx = to_tile<T, P>(load_raw<T, P, Full>(sxm, b, n, lane_m));
    Tm<P> lg;
    if constexpr (Pair) lg = to_tile<T, P>(load_raw<T, P, Full>(sgm, b, n, lane_m));

    // Both layouts of X (and G): the loaded one and its LDS transpose.
    PTm<P, Pair> a, at;
    {
      PTm<P, Pair> loaded;
      loaded.d = lx;
      if constexpr (Pair) loaded.u = lg;
      const PTm<P, Pair> other = ptranspose<P, Pair>(loaded, buf, lane);
      a.d = XL == kLoadCols ? other.d : lx;
      at.d = XL == kLoadCols ? lx : other.d;
      if constexpr (Pair) {
        a.u = GL == kLoadCols ? other.u : lg;
        at.u = GL == kLoadCols ? lg : other.u;
      }
    }

    int s;
    if (!squarings_from_estimate(norm_estimate<P, Pair>(a), s) && !exact_squarings<P, Pair>(a, buf, lane, s)) {
      // Non-finite entry: the whole matrix is NaN (csrc/MatrixExpSmall.cuh:318-331).
      Tm<P> nan;
#pragma unroll
      for (int r = 0; r < R; ++r) nan.v[r] = __builtin_nanf("");
      store_tile<T, P, Full>(args.out, b, n, lane_m, nan);
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

    // Degree-18 polynomial (csrc/MatrixExpSmall.cuh:83-106): A^2 = A.A,
    // A^3 = A.A^2, A^6 = A^3.A^3, A9 = B1.B5 + B4, T = B2 + (B3 + A9).A9.
    const PTm<P, Pair> a2 = pmm<P, Pair>(at, a);
    const PTm<P, Pair> a3 = pmm<P, Pair>(at, a2);
    const PTm<P, Pair> a6 = pmm<P, Pair>(ptranspose<P, Pair>(a3, buf, lane), a3);
    // The sums B1.B5 + B4, B3 + A9 and B2 + (..).A9 are formed after their
    // products, as in the reference: starting the MFMA accumulations from B4
    // and B2 instead raised the FP32 error 1.4-fold on average (measured over
    // config 5 against the FP64 result and the reference's own arithmetic).
    const PTm<P, Pair> b1t = ptranspose<P, Pair>(combine<0, P, Pair>(a, a2, a3, a6, id), buf, lane);
    const PTm<P, Pair> b5 = combine<4, P, Pair>(a, a2, a3, a6, id);
    const PTm<P, Pair> b1b5 = pmm<P, Pair>(b1t, b5);
    const PTm<P, Pair> a9 = padd<P, Pair>(b1b5, combine<3, P, Pair>(a, a2, a3, a6, id));
    const PTm<P, Pair> lhst = ptranspose<P, Pair>(padd<P, Pair>(combine<2, P, Pair>(a, a2, a3, a6, id), a9), buf, lane);
    const PTm<P, Pair> b2 = combine<1, P, Pair>(a, a2, a3, a6, id);
    PTm<P, Pair> res = padd<P, Pair>(b2, pmm<P, Pair>(lhst, a9));
    if constexpr (Pair) {
      // The last squaring forms only the U block (the output).
      for (int i = 1; i < s; ++i) res = pmm<P, Pair>(ptranspose<P, Pair>(res, buf, lane), res);
      if (s > 0) res = pmm<P, Pair, false>(ptranspose<P, Pair>(res, buf, lane), res);
    } else {
      for (int i = 0; i < s; ++i) res = pmm<P, Pair>(ptranspose<P, Pair>(res, buf, lane), res);
    }

    store_tile<T, P, Full>(args.out, b, n, lane_m, Pair ? res.u : res.d);
    if (lane == 0 && args.s_out) args.s_out[b] = s;
  }
}

template <typename T, int P, bool Pair, int XL, int GL, bool Full>
hipError_t launch_tile_l(const ExpmArgs& args, hipStream_t stream) {
  // P = 32: one matrix per wavefront (up to 2^24 workgroups, beyond which
  // wavefronts walk the batch with a grid stride), the hardware starting a
  // workgroup as another retires.  P = 16: four times the resident workgroups,
  // each walking two or three matrices, which spreads the per-wavefront setup
  // (C4 step 158.1 -> 155.0 and 159.2 -> 154.9 us against one matrix per
  // wavefront; 2x, 8x and 16x resident measured slower; P = 32 at 2x and 4x
  // slower than one per wavefront).
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_tile_kernel<T, P, Pair, XL, GL, Full>), 64);
  const int64_t cap = P == 16 ? 4 * resident : int64_t{1} << 24;
  const int64_t grid = args.batch < cap ? args.batch : cap;
  hipLaunchKernelGGL((expm_tile_kernel<T, P, Pair, XL, GL, Full>), dim3(static_cast<unsigned>(grid)), dim3(64), 0,
                     stream, args);
  return hipGetLastError();
}

int load_class(const Operand& op) { return (op.sr == 1 && op.sc != 1) ? kLoadCols : kLoadRows; }

template <typename T, int P, bool Pair, bool Full>
hipError_t launch_tile_f(const ExpmArgs& args, hipStream_t stream) {
  const int xl = load_class(args.x);
  if constexpr (Pair) {
    const int gl = load_class(args.g);
    if (xl == kLoadRows) {
      return gl == kLoadRows ? launch_tile_l<T, P, Pair, kLoadRows, kLoadRows, Full>(args, stream)
                             : launch_tile_l<T, P, Pair, kLoadRows, kLoadCols, Full>(args, stream);
    }
    return gl == kLoadRows ? launch_tile_l<T, P, Pair, kLoadCols, kLoadRows, Full>(args, stream)
                           : launch_tile_l<T, P, Pair, kLoadCols, kLoadCols, Full>(args, stream);
  } else {
    return xl == kLoadRows ? launch_tile_l<T, P, Pair, kLoadRows, kLoadRows, Full>(args, stream)
                           : launch_tile_l<T, P, Pair, kLoadCols, kLoadRows, Full>(args, stream);
  }
}

template <typename T, int P, bool Pair>
hipError_t launch_tile_tp(const ExpmArgs& args, hipStream_t stream) {
  return args.n == P ? launch_tile_f<T, P, Pair, true>(args, stream) : launch_tile_f<T, P, Pair, false>(args, stream);
}

template <typename T, bool Pair>
hipError_t launch_tile_t(const ExpmArgs& args, int P, hipStream_t stream) {
  return P == 16 ? launch_tile_tp<T, 16, Pair>(args, stream) : launch_tile_tp<T, 32, Pair>(args, stream);
}

// Buffer addressing needs non-negative in-matrix strides and a per-matrix
// footprint below 2^31 bytes.
bool addressable(const Operand& op, int n, int es) {
  if (op.sr < 0 || op.sc < 0) return false;
  const int64_t limit = (int64_t{1} << 31) / es;
  if (op.sr >= limit || op.sc >= limit) return false;
  return (n - 1) * (op.sr + op.sc) + 1 < limit;
}

}  // namespace

hipError_t launch_tile(const ExpmArgs& args, int dtype, int P, bool pair, hipStream_t stream) {
  const int es = dtype == F32::code ? 4 : 2;
  if (!addressable(args.x, args.n, es) || (pair && !addressable(args.g, args.n, es)))
    return launch_generic(args, dtype, P, pair, stream);
  if (dtype == F32::code) return pair ? launch_tile_t<F32, true>(args, P, stream) : launch_tile_t<F32, false>(args, P, stream);
  if (dtype == BF16::code) return pair ? launch_tile_t<BF16, true>(args, P, stream) : launch_tile_t<BF16, false>(args, P, stream);
  return pair ? launch_tile_t<F16, true>(args, P, stream) : launch_tile_t<F16, false>(args, P, stream);
}

}  // namespace fh

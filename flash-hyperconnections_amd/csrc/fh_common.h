// Shared device-side pieces of the gfx950 small-matrix exponential kernels:
// kernel argument block, element load/store with exact dtype conversion, the
// degree-18 coefficient table and the squaring-count rule.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fh {

// Squaring threshold of the degree-18 polynomial (reference
// csrc/MatrixExpSmall.cuh:14).
constexpr double kTheta18 = 3.010066362817634;

// Coefficients of the Bader-Blanes-Casas (2019) degree-18 evaluation, as FP32
// literals (reference csrc/MatrixExpSmall.cuh:89-103).  Row k is B(k+1);
// columns multiply (I, A, A^2, A^3, A^6).
#define FH_COEF_TABLE                                                                                   \
  {                                                                                                     \
    {0.f, -0.10036558103014462f, -0.008029246482411570f, -0.000892138498045730f, 0.f},                \
    {0.f, 0.39784974949645076f, 1.36783778460411719f, 0.49828962252538268f,                            \
     -0.00063789819459247233f},                                                                        \
    {-10.96763960529620626f, 1.68015813878906197f, 0.05717798464788655f, -0.00698210122488052f,        \
     3.349750170860705e-05f},                                                                          \
    {-0.09043168323908106f, -0.06764045190713819f, 0.06759613017740597f, 0.02955525704293155f,         \
     -1.391802575160607e-05f},                                                                         \
    {0.f, 0.f, -0.09233646193671186f, -0.01693649390020817f, -1.400867981820361e-05f},                \
  }

__device__ constexpr float kCoef[5][5] = FH_COEF_TABLE;

// +0 held in a VGPR the compiler cannot see through.  A combine's first term
// fmaf(c, x, +0) with the +0 constant-folded has to take the coefficient from
// an SGPR (gfx9's three-operand encoding carries no literal); with +0 in a
// VGPR it encodes as v_fmamk_f32 with the coefficient as a literal, same
// operation, same bits.  In isolation gfx950 issues the SGPR form ~1.6x
// slower (4.7 against 2.9 cycles per instruction at two wavefronts per SIMD);
// in the P = 8 forward kernel the literal form measured 5% faster, in the
// P = 4 and tile kernels no faster, which keep the SGPR form.
__device__ __forceinline__ float vgpr_zero() {
  float z;
  asm("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// Element types, tagged by the reference's dtype codes
// (csrc/matrix_exp.cu:17: 0 = float32, 1 = bfloat16, 2 = float16).
struct F32 {
  using storage = float;
  static constexpr int code = 0;
};
struct BF16 {
  using storage = uint16_t;
  static constexpr int code = 1;
};
struct F16 {
  using storage = _Float16;
  static constexpr int code = 2;
};

// One [batch, n, n] operand read through element strides.  `sign` is -1 for
// a lazily negated tensor view and +1 otherwise (multiplying by it is exact).
// `vec` tells the P == 4 and P == 8 kernels that every row (kVecRows:
// sc == 1) or every column (kVecCols: sr == 1) of a 4 x 4 or 8 x 8 matrix is
// made of aligned 4-element vectors; the host sets it only when n is 4 or 8
// and the alignment holds.  `dense` adds that the matrices themselves are
// packed (n * n elements apart, rows or columns n apart), so consecutive
// matrices are one contiguous, 16-byte aligned block.
constexpr int kVecNone = 0;
constexpr int kVecRows = 1;
constexpr int kVecCols = 2;
struct Operand {
  const void* data;
  int64_t sb, sr, sc;
  float sign;
  int vec;
  int dense;
};

struct ExpmArgs {
  Operand x;        // the matrix X
  Operand g;        // the Frechet direction G (unused by the forward)
  void* out;        // contiguous [batch, n, n] in the input dtype
  int32_t* s_out;   // optional per-matrix squaring count (-1: non-finite)
  int64_t batch;
  int n;
};

template <typename T>
__device__ __forceinline__ float to_f32(typename T::storage v);
template <>
__device__ __forceinline__ float to_f32<F32>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<F16>(_Float16 v) { return static_cast<float>(v); }
template <>
__device__ __forceinline__ float to_f32<BF16>(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// FP32 -> storage type, round to nearest even (the reference stores through
// c10::BFloat16(float) / c10::Half(float), csrc/MatrixExpSmall.cuh:108-112).
template <typename T>
__device__ __forceinline__ typename T::storage from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<F32>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 from_f32<F16>(float v) { return static_cast<_Float16>(v); }
template <>
__device__ __forceinline__ uint16_t from_f32<BF16>(float v) {
  if (v != v) return 0x7FC0;
  uint32_t u = __float_as_uint(v);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Logical element (r, c) of matrix b, converted exactly to FP32.
template <typename T>
__device__ __forceinline__ float load_elem(const Operand& op, int64_t b, int r, int c) {
  const auto* p = static_cast<const typename T::storage*>(op.data);
  return to_f32<T>(p[b * op.sb + static_cast<int64_t>(r) * op.sr + static_cast<int64_t>(c) * op.sc]) * op.sign;
}

// Same without the view's sign (kernels that fold the sign into a later
// exact multiply).
template <typename T>
__device__ __forceinline__ float load_elem_nosign(const Operand& op, int64_t b, int r, int c) {
  const auto* p = static_cast<const typename T::storage*>(op.data);
  return to_f32<T>(p[b * op.sb + static_cast<int64_t>(r) * op.sr + static_cast<int64_t>(c) * op.sc]);
}

template <typename T>
__device__ __forceinline__ void store_elem(void* out, int64_t idx, float v) {
  static_cast<typename T::storage*>(out)[idx] = from_f32<T>(v);
}

// ceil(log2(q)) through the library log2; kept out of line because only the
// rare band below needs it.
static __device__ __attribute__((noinline)) int ceil_log2_library(double q) { return static_cast<int>(ceil(log2(q))); }

// s = norm > theta18 ? ceil(log2(norm / theta18)) : 0, in double (reference
// csrc/MatrixExpSmall.cuh:154, :356).  For q = norm/theta18 = m * 2^e with
// m in [0.5, 1): ceil(log2 q) is e - 1 when m == 0.5 and e otherwise, and any
// log2 accurate to better than 2^-40 relative returns the same integer ceiling
// unless q lies within 2^-40 above a power of two; only that band calls log2.
__device__ __forceinline__ int squarings_from_norm(double norm) {
  if (!(norm > kTheta18)) return 0;
  const double q = norm / kTheta18;
  int e;
  const double m = frexp(q, &e);
  if (m == 0.5) return e - 1;
  if (m < 0.5 + 0x1p-41) return ceil_log2_library(q);
  return e;
}

// s from an FP32 estimate of the norm whose relative error is below 2^-18.
// s(norm) is monotone and steps only where norm / theta18 crosses a power of
// two, so when the estimate keeps q = norm / theta18 at least 2^-16 (relative)
// away from every power of two, the exact FP64 norm lies on the same step and
// has the same s.  Returns false -- only the exact norm can decide -- inside
// those bands and for huge or non-finite estimates.
__device__ __forceinline__ bool squarings_from_estimate(float norm, int& s) {
  if (!(norm < 0x1p120f)) return false;
  constexpr float kInvTheta = static_cast<float>(1.0 / kTheta18);
  const float q = norm * kInvTheta;
  if (q <= 0.5f) {
    s = 0;
    return true;
  }
  int e;
  const float m = __builtin_frexpf(q, &e);
  if (m < 0.5f + 0x1p-16f || m > 1.f - 0x1p-16f) return false;
  s = e > 0 ? e : 0;
  return true;
}

// Raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

// An offset no footprint reaches: buffer loads there return 0, stores drop.
constexpr int32_t kOutOfRange = static_cast<int32_t>(0x80000000u);

// Cache policy of result stores: the nontemporal hint ("nt", bit 1 on
// gfx950).  Nothing in a launch reads its outputs back; with the hint the
// P = 4 forward at config 2 ran 24.6 -> 22.9 us and its Frechet kernel
// 55.9 -> 52.4 us (same process, alternating).  Loads keep the default
// policy: the backward re-reads the forward's input, which the hint would
// stop the caches from keeping.
constexpr int kNontemporal = 2;

// A buffer store of more than 8 bytes reads its data registers after it
// issues; the compiler keeps the next instruction from overwriting them only
// when the store's scalar offset is the constant 0 (its hazard check exempts
// stores with an SGPR offset), and on gfx950 such an overwrite was observed to
// reach memory (the first dword of a 16-byte nontemporal store replaced by the
// following instruction's result).  So 16-byte stores take their whole offset
// in the VGPR offset and pass this as the scalar offset.
constexpr int32_t kStoreSOffset = 0;

// Element I/O through a buffer resource, keeping the storage bits (`raw_t`)
// separate from the conversion so that a prefetch never waits for its data.
template <typename T>
struct ElemIO;
template <>
struct ElemIO<F32> {
  using raw_t = uint32_t;
  static constexpr int bytes = 4;
  __device__ static __forceinline__ raw_t load(__amdgpu_buffer_rsrc_t rs, int32_t voff, int32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0);
  }
  __device__ static __forceinline__ float value(raw_t v) { return __uint_as_float(v); }
  template <int Policy = 0>
  __device__ static __forceinline__ void store(float v, __amdgpu_buffer_rsrc_t rs, int32_t voff, int32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rs, voff, soff, Policy);
  }
};
template <>
struct ElemIO<F16> {
  using raw_t = uint16_t;
  static constexpr int bytes = 2;
  __device__ static __forceinline__ raw_t load(__amdgpu_buffer_rsrc_t rs, int32_t voff, int32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff, 0);
  }
  __device__ static __forceinline__ float value(raw_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  }
  template <int Policy = 0>
  __device__ static __forceinline__ void store(float v, __amdgpu_buffer_rsrc_t rs, int32_t voff, int32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<F16>(v)), rs, voff, soff, Policy);
  }
};
template <>
struct ElemIO<BF16> {
  using raw_t = uint16_t;
  static constexpr int bytes = 2;
  __device__ static __forceinline__ raw_t load(__amdgpu_buffer_rsrc_t rs, int32_t voff, int32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff, 0);
  }
  __device__ static __forceinline__ float value(raw_t v) { return to_f32<BF16>(v); }
  template <int Policy = 0>
  __device__ static __forceinline__ void store(float v, __amdgpu_buffer_rsrc_t rs, int32_t voff, int32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b16(from_f32<BF16>(v), rs, voff, soff, Policy);
  }
};

__device__ __forceinline__ bool finite_f32(float v) { return __builtin_isfinite(v); }

// ---- buffer-to-LDS loads ------------------------------------------------------

typedef uint32_t U32x4 __attribute__((ext_vector_type(4)));

// Buffer-to-LDS load of 16 bytes per lane: lane l's bytes land at LDS byte
// address lds_addr + 16 l.  Written as assembly so that the compiler's wait
// insertion does not make every LDS read wait for these loads (it cannot tell
// LDS areas apart); wait_vm<N>() orders them instead.  `rsrc` is the buffer
// resource as four words.
__device__ __forceinline__ void lds_load16(U32x4 rsrc, uint32_t lds_addr, int32_t voff, int32_t soff) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" : : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

// Resource words of make_rsrc(base, 0x7FFFFFFF): base address, stride 0,
// num_records, and the same fourth word.
__device__ __forceinline__ U32x4 rsrc_words(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return U32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xFFFFu, 0x7FFFFFFFu, 0x00020000u};
}

// s_waitcnt vmcnt(N): at most N vector memory operations of this wavefront
// outstanding.  Loads complete in issue order, so this waits for every load
// issued before the last N loads.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// s_waitcnt lgkmcnt(0): every LDS access this wavefront issued is complete.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Lanes below this one whose bit is set in `mask`.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}

}  // namespace fh

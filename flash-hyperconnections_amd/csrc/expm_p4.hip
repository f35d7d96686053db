// P == 4 kernel (n = 2, 3, 4): one matrix per lane, 64 matrices per
// wavefront.
//
// Each lane keeps its whole 4 x 4 matrix (16 VGPRs; the Frechet kernel keeps
// the D and U blocks, 32 VGPRs) and every product is 64 plain FP32 FMAs with
// compile-time register indices -- no cross-lane traffic, no transposes.  The
// per-matrix scalar work (norm, squaring count, scaling) is done once per
// matrix rather than once per row.
//
// What bounds it on gfx950 (measured): wave64 FP32 VALU instructions issue
// every ~2.5-3 cycles per SIMD with two or more wavefronts on it (~5 cycles
// with one), FP32 MFMA does not overlap VALU work on the same SIMD, and a VALU
// instruction with 16 or fewer active lanes costs ~5x a full one.  So the
// kernel is shaped to issue as few VALU instructions as possible, all with
// full exec masks:
//  * operand classes (row / column vectors, dense 64-matrix blocks) are
//    template parameters, so no register shuffles join alternative load paths;
//  * loads and stores go through buffer resources with the group offset in an
//    SGPR: no VALU address arithmetic;
//  * raw storage bytes are staged as 16-byte tuples until the group's turn, so
//    a prefetch stays in flight across the previous group's polynomial and
//    feeds LDS writes without repacking;
//  * squarings run over the full wavefront on ping-pong register sets; each
//    lane keeps (by a select) the result of its own last squaring, and the
//    wavefront's last squaring forms only the block the output needs.
// The one partial group of a batch (B % 64 matrices) takes a separate, cold
// path with per-element loads and stores.
//
// Arithmetic is the reference's, element by element (csrc/MatrixExpSmall.cuh:
// 22-106): product entries accumulate k = 0..3 with fmaf from +0, Frechet U
// blocks sum D.U and U.D separately and add them, combines are the
// contracted chain c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6 with its zero
// coefficients skipped.  Results are bit-identical to that evaluation up to
// the sign of zero results.  Nothing a matrix computes depends on the batch
// size or on its position in the batch.
#include "p4_lane.h"

namespace fh {
namespace {

using namespace p4;

// ---- operand staging --------------------------------------------------------
//
// Layout classes (compile time, set by the host for n == 4): kVecRows -- each
// row is one aligned 4-element vector (sc == 1); kVecCols -- each column is
// (sr == 1); kVecNone -- element loads through the strides, n <= 4, padded.
// Dense (compile time as well): the 64 matrices of a group are one contiguous
// block of 64 * 16 elements in the class's memory order.

// Raw storage of one lane's share of a group: C 16-byte tuples, where C is the
// number of tuples one matrix spans (4 in FP32, 2 in FP16/BF16).
template <typename T>
struct Raw {
  static constexpr int C = static_cast<int>(sizeof(typename T::storage));
  uint4 q[C];
};

// Dense group: tuples lane, lane + 64, ... of the group's contiguous block, so
// that each load instruction reads 1 KB of consecutive memory.  `group_bytes`
// is the uniform byte offset of the group in the operand.
template <typename T>
__device__ __forceinline__ Raw<T> load_dense(__amdgpu_buffer_rsrc_t rs, int lane, int32_t group_bytes) {
  Raw<T> r;
#pragma unroll
  for (int c = 0; c < Raw<T>::C; ++c) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * lane, group_bytes + 1024 * c, 0);
    r.q[c] = make_uint4(v[0], v[1], v[2], v[3]);
  }
  return r;
}

// Per-lane vectors: the matrix's four rows (kVecRows) or columns (kVecCols),
// 4 elements each, at byte offset `mat_bytes` (uniform part `group_bytes`).
template <typename T, int L>
__device__ __forceinline__ Raw<T> load_lane(__amdgpu_buffer_rsrc_t rs, int32_t mat_bytes, int32_t step_bytes,
                                            int32_t group_bytes) {
  Raw<T> r;
  if constexpr (sizeof(typename T::storage) == 4) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(rs, mat_bytes + v * step_bytes, group_bytes, 0);
      r.q[v] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const auto x0 = __builtin_amdgcn_raw_buffer_load_b64(rs, mat_bytes + (2 * h) * step_bytes, group_bytes, 0);
      const auto x1 = __builtin_amdgcn_raw_buffer_load_b64(rs, mat_bytes + (2 * h + 1) * step_bytes, group_bytes, 0);
      r.q[h] = make_uint4(x0[0], x0[1], x1[0], x1[1]);
    }
  }
  return r;
}


// Routes a dense group's tuples through the wavefront's LDS tile so that each
// lane ends up with its own matrix: tuple c of matrix m goes to byte
// c * 1040 + 16 * m (rows of 64 tuples padded by 16 bytes, so that both the
// scattered writes and the per-lane reads are free of bank conflicts).
constexpr int kDenseRowBytes = 1024 + 16;

template <typename T>
__device__ __forceinline__ void dense_to_lane(Raw<T>& r, char* tile, int lane) {
  constexpr int C = Raw<T>::C;
#pragma unroll
  for (int q = 0; q < C; ++q) {
    const int g = q * 64 + lane;  // tuple g of the block: matrix g / C, tuple g % C of it
    *reinterpret_cast<uint4*>(tile + (g % C) * kDenseRowBytes + 16 * (g / C)) = r.q[q];
  }
  lds_order();
#pragma unroll
  for (int c = 0; c < C; ++c) r.q[c] = *reinterpret_cast<const uint4*>(tile + c * kDenseRowBytes + 16 * lane);
  lds_order();
}

// Row-major FP32 matrix (without the view's sign) from one matrix's tuples in
// the class's memory order (rows: e = 4 * row + col; columns: e = 4 * col + row).
template <typename T, int L>
__device__ __forceinline__ M4 decode(const Raw<T>& r) {
  using S = typename T::storage;
  M4 m;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float v;
    if constexpr (sizeof(S) == 4) {
      const uint4& t = r.q[e >> 2];
      const uint32_t w = (e & 3) == 0 ? t.x : (e & 3) == 1 ? t.y : (e & 3) == 2 ? t.z : t.w;
      v = __uint_as_float(w);
    } else {
      const uint4& t = r.q[e >> 3];
      const int k = (e >> 1) & 3;
      const uint32_t w = k == 0 ? t.x : k == 1 ? t.y : k == 2 ? t.z : t.w;
      const uint16_t h = static_cast<uint16_t>(w >> (16 * (e & 1)));
      v = to_f32<T>(__builtin_bit_cast(S, h));
    }
    m.v[L == kVecRows ? e : 4 * (e & 3) + (e >> 2)] = v;
  }
  return m;
}


constexpr int kP4Waves = 4;       // wavefronts per workgroup
constexpr int kStageStride = 17;  // floats per matrix in the LDS staging tile (odd: conflict-free)

// Per-wavefront LDS tile: the store staging area and, in turn, one (forward)
// or two (Frechet: X and G) dense-group routing areas of 4 x 1040 bytes.
template <bool Pair>
constexpr int kTileBytes = (Pair ? 2 : 1) * 4 * kDenseRowBytes > 4 * 64 * kStageStride
                               ? (Pair ? 2 : 1) * 4 * kDenseRowBytes
                               : 4 * 64 * kStageStride;

// Stores the 64 matrices of a full group (n == 4) through the wavefront's LDS
// tile so that the global stores are coalesced: lane l has written its matrix
// with element-wise LDS stores (stage_lane: stride 17, no bank conflicts);
// then in each of four passes every lane stores 4 consecutive elements, pass p
// covering elements [256 p, 256 p + 256) of the group's contiguous block.
__device__ __forceinline__ void stage_lane(float* tile, int lane, const M4& m) {
#pragma unroll
  for (int e = 0; e < 16; ++e) tile[lane * kStageStride + e] = m.v[e];
}

template <typename T>
__device__ __forceinline__ void store_group(__amdgpu_buffer_rsrc_t out, int32_t group_bytes, int lane, float* tile) {
  lds_order();
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int f = pass * 256 + 4 * lane;  // first element of this lane's 4 in the group block
    const int mat = f >> 4;
    const int e = f & 15;
    const float v0 = tile[mat * kStageStride + e];
    const float v1 = tile[mat * kStageStride + e + 1];
    const float v2 = tile[mat * kStageStride + e + 2];
    const float v3 = tile[mat * kStageStride + e + 3];
    if constexpr (sizeof(typename T::storage) == 4) {
      const U32x4 w = {__float_as_uint(v0), __float_as_uint(v1), __float_as_uint(v2), __float_as_uint(v3)};
      __builtin_amdgcn_raw_buffer_store_b128(w, out, group_bytes + 4 * f, kStoreSOffset, kNontemporal);
    } else {
      const uint32_t lo = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v0))) |
                          (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v1))) << 16);
      const uint32_t hi = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v2))) |
                          (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v3))) << 16);
      const U32x2 w = {lo, hi};
      __builtin_amdgcn_raw_buffer_store_b64(w, out, 2 * f, group_bytes, kNontemporal);
    }
  }
  lds_order();
}

// The partial last group (lanes with b < batch) and every group of an
// element-class operand: per-element loads and stores through the strides.
template <typename T, bool Pair>
__device__ __forceinline__ void expm_group_elements(const ExpmArgs& args, int64_t group, int lane) {
  const int64_t b = group * 64 + lane;
  const bool valid = b < args.batch;
  PM<Pair> cur;
  if (valid) {
    cur.d = load_elements<T>(args.x, b, args.n);
    if constexpr (Pair) cur.u = load_elements<T>(args.g, b, args.n);
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      cur.d.v[e] = 0.f;
      if constexpr (Pair) cur.u.v[e] = 0.f;
    }
  }
  M4 res;
  const int s = expm_lane<Pair>(cur, args.x.sign, args.g.sign, [&](const M4& out) { res = out; });
  if (s < 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) res.v[e] = __builtin_nanf("");
  }
  if (valid) {
    store_elements<T>(args.out, b, args.n, res);
    if (args.s_out) args.s_out[b] = s;
  }
}

// Per-operand addressing of the vector classes: a buffer resource over the
// operand, the lane's byte offset within a group and the group's byte stride.
struct VecSrc {
  __amdgpu_buffer_rsrc_t rs;
  int32_t lane_bytes;   // dense: unused; per lane: lane * sb * es
  int32_t step_bytes;   // per lane: bytes between the four vectors (sr or sc)
  int32_t group_bytes;  // bytes between consecutive groups (64 * sb * es)
};

template <typename T>
__device__ __forceinline__ VecSrc make_vec_src(const Operand& op, int L, int lane) {
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  VecSrc v;
  v.rs = make_rsrc(op.data, 0x7FFFFFFFu);
  v.lane_bytes = static_cast<int32_t>(lane * op.sb * es);
  v.step_bytes = static_cast<int32_t>((L == kVecRows ? op.sr : op.sc) * es);
  v.group_bytes = static_cast<int32_t>(64 * op.sb * es);
  return v;
}

template <typename T, int L, bool Dense>
__device__ __forceinline__ Raw<T> load_vec(const VecSrc& src, int lane, int32_t group) {
  const int32_t off = group * src.group_bytes;
  if constexpr (Dense) {
    return load_dense<T>(src.rs, lane, off);
  } else {
    return load_lane<T, L>(src.rs, src.lane_bytes, src.step_bytes, off);
  }
}

// Persistent kernel over the full groups of a vector-class batch (n == 4):
// each wavefront walks 64-matrix groups with a grid stride and keeps the next
// group's loads in flight while it computes.  XD / GD: the operand is dense.
template <typename T, bool Pair, int XL, int GL, bool XD, bool GD>
__global__ __launch_bounds__(64 * kP4Waves) __attribute__((amdgpu_waves_per_eu(Pair ? 2 : 4, 8))) void expm_p4_kernel(
    ExpmArgs args) {
  __shared__ __attribute__((aligned(16))) char tile_mem[kP4Waves][kTileBytes<Pair>];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: offsets stay in SGPRs
  char* tile = tile_mem[wave];
  // Groups fit in 32 bits: the host takes this kernel only for operands below 2 GiB.
  const int32_t full = static_cast<int32_t>(args.batch / 64);
  const int32_t stride = static_cast<int32_t>(gridDim.x) * kP4Waves;
  int32_t group = static_cast<int32_t>(blockIdx.x) * kP4Waves + wave;
  constexpr int es = static_cast<int>(sizeof(typename T::storage));

  const VecSrc sx = make_vec_src<T>(args.x, XL, lane);
  VecSrc sg = sx;
  if constexpr (Pair) sg = make_vec_src<T>(args.g, GL, lane);
  const __amdgpu_buffer_rsrc_t out_rs = make_rsrc(args.out, 0x7FFFFFFFu);

  Raw<T> nx, ng;
  if (group < full) {
    nx = load_vec<T, XL, XD>(sx, lane, group);
    if constexpr (Pair) ng = load_vec<T, GL, GD>(sg, lane, group);
  }
  for (; group < full; group += stride) {
    Raw<T> rx = nx, rg = ng;
    if constexpr (XD) dense_to_lane<T>(rx, tile, lane);
    if constexpr (Pair && GD) dense_to_lane<T>(rg, tile + 4 * kDenseRowBytes, lane);
    PM<Pair> cur;
    cur.d = decode<T, XL>(rx);
    if constexpr (Pair) cur.u = decode<T, GL>(rg);
    // Next group's loads, in flight across this group's polynomial; the last
    // round reloads the final group instead of branching around the loads.
    const int32_t next = group + stride < full ? group + stride : full - 1;
    nx = load_vec<T, XL, XD>(sx, lane, next);
    if constexpr (Pair) ng = load_vec<T, GL, GD>(sg, lane, next);
    float* stage = reinterpret_cast<float*>(tile);
    const int s = expm_lane<Pair>(cur, args.x.sign, args.g.sign, [&](const M4& out) { stage_lane(stage, lane, out); });
    if (s < 0) {  // rare: overwrite the staged block with NaN
      M4 nan;
#pragma unroll
      for (int e = 0; e < 16; ++e) nan.v[e] = __builtin_nanf("");
      stage_lane(stage, lane, nan);
    }
    store_group<T>(out_rs, group * 64 * 16 * es, lane, stage);
    if (args.s_out) args.s_out[static_cast<int64_t>(group) * 64 + lane] = s;
  }
  // The partial last group, if any, belongs to the wavefront whose walk reaches it.
  if (group == full && static_cast<int64_t>(full) * 64 < args.batch) expm_group_elements<T, Pair>(args, group, lane);
}

// ---- dense operands: groups loaded straight into LDS ------------------------
//
// For dense operands the groups go from HBM to the wavefront's LDS with
// buffer-to-LDS loads, no registers involved, a group ahead in a two-slot
// ring when a wavefront walks several groups (the Frechet kernel's persistent
// grid; the forward's grid gives each wavefront one group, so its second slot
// stays idle).  Load instruction c of a group has lane l fetch tuple C l + c of the
// 64-matrix block, so that it writes LDS row c with matrix l's tuple c at byte
// 16 l: the padded, conflict-free layout each lane reads its own matrix from.
// A slot is reused for the group's staged results once its inputs are read.

// One operand's group block into LDS rows c * 1040 (the dense_to_lane layout).
template <typename T>
__device__ __forceinline__ void load_group_to_lds(U32x4 rs, uint32_t lds_addr, int32_t group_bytes, int lane) {
  constexpr int C = Raw<T>::C;
#pragma unroll
  for (int c = 0; c < C; ++c) lds_load16(rs, lds_addr + c * kDenseRowBytes, 16 * C * lane, group_bytes + 16 * c);
}

template <typename T>
__device__ __forceinline__ Raw<T> read_lane_tuples(const char* area, int lane) {
  Raw<T> r;
#pragma unroll
  for (int c = 0; c < Raw<T>::C; ++c) r.q[c] = *reinterpret_cast<const uint4*>(area + c * kDenseRowBytes + 16 * lane);
  return r;
}

template <typename T, bool Pair>
struct DmaSlot {
  static constexpr int kArea = Raw<T>::C * kDenseRowBytes;
  static constexpr int kIn = (Pair ? 2 : 1) * kArea;
  static constexpr int kStage = 64 * kStageStride * 4;
  static constexpr int kBytes = kIn > kStage ? kIn : kStage;  // inputs, then the staged results
};

// Persistent kernel over the full groups of a batch whose operands are all
// dense (n == 4).
template <typename T, bool Pair, int XL, int GL>
__global__ __launch_bounds__(64 * kP4Waves) __attribute__((amdgpu_waves_per_eu(Pair ? 2 : 4, 8))) void expm_p4_dma_kernel(
    ExpmArgs args) {
  using Slot = DmaSlot<T, Pair>;
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  constexpr int kLoads = Raw<T>::C * (Pair ? 2 : 1);  // load instructions per group
  __shared__ __attribute__((aligned(16))) char tile_mem[kP4Waves][2][Slot::kBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Groups fit in 32 bits: the host takes this kernel only for operands below 2 GiB.
  const int32_t full = static_cast<int32_t>(args.batch / 64);
  const int32_t stride = static_cast<int32_t>(gridDim.x) * kP4Waves;
  int32_t group = static_cast<int32_t>(blockIdx.x) * kP4Waves + wave;
  const U32x4 xs = rsrc_words(args.x.data);
  const U32x4 gs = rsrc_words(Pair ? args.g.data : args.x.data);
  const __amdgpu_buffer_rsrc_t out_rs = make_rsrc(args.out, 0x7FFFFFFFu);
  constexpr int32_t kGroupBytes = 64 * 16 * es;
  auto issue = [&](int32_t g, char* slot) {
    const uint32_t a = lds_address(slot);
    load_group_to_lds<T>(xs, a, g * kGroupBytes, lane);
    if constexpr (Pair) load_group_to_lds<T>(gs, a + Slot::kArea, g * kGroupBytes, lane);
  };
  int which = 0;
  if (group < full) issue(group, tile_mem[wave][0]);
  for (; group < full; group += stride) {
    char* slot = tile_mem[wave][which];
    // The next group's loads go to the other slot (its results were read out
    // for the stores of the previous round); then wait for this group's.
    if (group + stride < full) {
      issue(group + stride, tile_mem[wave][which ^ 1]);
      wait_vm<kLoads>();
    } else {
      wait_vm<0>();
    }
    lds_order();
    PM<Pair> cur;
    cur.d = decode<T, XL>(read_lane_tuples<T>(slot, lane));
    if constexpr (Pair) cur.u = decode<T, GL>(read_lane_tuples<T>(slot + Slot::kArea, lane));
    lds_order();  // inputs read before the staged results overwrite the slot
    float* stage = reinterpret_cast<float*>(slot);
    const int s = expm_lane<Pair>(cur, args.x.sign, args.g.sign, [&](const M4& out) { stage_lane(stage, lane, out); });
    if (s < 0) {  // rare: overwrite the staged block with NaN
      M4 nan;
#pragma unroll
      for (int e = 0; e < 16; ++e) nan.v[e] = __builtin_nanf("");
      stage_lane(stage, lane, nan);
    }
    store_group<T>(out_rs, group * kGroupBytes, lane, stage);
    if (args.s_out) args.s_out[static_cast<int64_t>(group) * 64 + lane] = s;
    which ^= 1;
  }
  // The partial last group, if any, belongs to the wavefront whose walk reaches it.
  if (group == full && static_cast<int64_t>(full) * 64 < args.batch) expm_group_elements<T, Pair>(args, group, lane);
}

// ---- 2-byte dtypes: batches of groups ordered by squaring count -------------
//
// A wavefront squares up to the largest count among its 64 matrices, so when
// counts spread (inputs over several decades of norm) most of a group's
// squaring rounds run for a few lanes.  For FP16/BF16 a wavefront's LDS holds
// a batch of G groups' inputs per slot (SortSlot): the kernel computes the
// count of all 64 G matrices, ranks them by (count, position) with a counting
// sort over ballots, and runs G rounds of 64 in rank order, so the early
// rounds square only up to low counts.  Each matrix's result (already in the
// output dtype, 32 bytes) replaces its own first input tuples in the slot,
// from where the batch's groups are stored coalesced.  Which lane computes a
// matrix does not change what it computes, so results are the unsorted
// kernel's.

// Groups per batch and LDS slots per wavefront: two slots (the next batch
// loads while this one computes) of two groups each.  Batches of four groups
// in one slot (the same LDS) for the forward, which gives each wavefront one
// batch, were bit-identical but no faster (config 3 forward 23.9 -> 24.3 us,
// same process, alternating): half as many wavefronts and a longer ranking
// loop outweigh the squaring rounds saved.
template <typename T, bool Pair>
struct SortSlot {
  static_assert(sizeof(typename T::storage) == 2, "batches of groups fit the LDS budget for 2-byte dtypes only");
  static constexpr int G = 2;                            // groups per batch
  static constexpr int kSlots = 2;                       // slots per wavefront
  static constexpr int C = Raw<T>::C;                    // tuples per matrix (2)
  static constexpr int kArea = C * kDenseRowBytes;       // one operand of one group
  static constexpr int kGroup = (Pair ? 2 : 1) * kArea;  // one group's inputs
  static constexpr int kBytes = G * kGroup;              // the batch's groups
};

// Matrix m's tuples in an operand area of the slot (rows c * 1040, byte 16 m).
template <typename T>
__device__ __forceinline__ Raw<T> read_tuples_at(const char* area, int m) {
  Raw<T> r;
#pragma unroll
  for (int c = 0; c < Raw<T>::C; ++c) r.q[c] = *reinterpret_cast<const uint4*>(area + c * kDenseRowBytes + 16 * m);
  return r;
}

// A row-major result in the 2-byte output dtype, written over matrix m's input
// tuples: tuple c holds output elements 8c .. 8c + 7.  BF16 goes through
// gfx950's packed conversion (round to nearest even, bit-identical to the
// software rounding for every non-NaN value) unless a lane of the wavefront
// holds a NaN, which the software rounding writes as the reference's 0x7FC0
// whatever its sign and payload.  `nan_free`: the caller knows no lane can.
// FP16 always takes the packed conversion, which gives the scalar
// conversion's bits for every input (NaNs included; measured on gfx950).
typedef __bf16 BF16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 F16x2 __attribute__((ext_vector_type(2)));
typedef float F32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ void write_result_at(char* area, int m, const M4& v, bool nan_free) {
  bool packed = __is_same(T, F16);
  if constexpr (__is_same(T, BF16)) {
    packed = nan_free;
    if (!packed) {
      float t = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) t += __builtin_fabsf(v.v[e]);  // NaN exactly when an entry is
      packed = !any_lane(t != t);
    }
  }
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = 8 * c + 2 * k;
      if (packed) {
        const F32x2 f = {v.v[e], v.v[e + 1]};
        if constexpr (__is_same(T, F16)) {
          w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, F16x2));
        } else {
          w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, BF16x2));
        }
      } else {
        w[k] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v.v[e]))) |
               (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v.v[e + 1]))) << 16);
      }
    }
    *reinterpret_cast<uint4*>(area + c * kDenseRowBytes + 16 * m) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// With every count at most 4 the wavefront's (augmented) norms are at most
// 16 theta18 < 49: the polynomial's intermediates stay below ~1e16 and the
// squarings below ~e^49 (every partial sum is bounded by the product of the
// factors' norms), so no entry overflows and no NaN can arise; a non-finite
// matrix (count -1) is overwritten by the default NaN, which both roundings
// write as 0x7FC0.
constexpr int kNanFreeCount = 4;

// Units of a 2-byte dense batch (n == 4) for expm_p4_sort_kernel: the sorted
// batches of G full groups, then one unit per group left over (the full
// groups after the last batch and a partial last group), so that no
// wavefront takes more than one of them.
template <typename T, bool Pair>
__host__ __device__ constexpr int64_t sort_units(int64_t batch) {
  constexpr int G = SortSlot<T, Pair>::G;
  const int64_t full = batch / 64;
  return full / G + full % G + (full * 64 < batch ? 1 : 0);
}

// Kernel over batches of G full groups of a 2-byte dense batch (n == 4):
// batch q is groups G q .. G q + G - 1; the units after the last batch are the
// left-over groups, one per unit.
template <typename T, bool Pair, int XL, int GL>
__global__ __launch_bounds__(64 * kP4Waves) __attribute__((amdgpu_waves_per_eu(Pair ? 2 : 4, 8))) void expm_p4_sort_kernel(
    ExpmArgs args) {
  using Slot = SortSlot<T, Pair>;
  constexpr int G = Slot::G;
  constexpr int C = Slot::C;
  constexpr int es = 2;
  constexpr int kLoads = G * C * (Pair ? 2 : 1);  // load instructions per batch
  constexpr int32_t kGroupBytes = 64 * 16 * es;
  __shared__ __attribute__((aligned(16))) char tile_mem[kP4Waves][Slot::kSlots][Slot::kBytes];
  __shared__ uint8_t order_mem[kP4Waves][G * 64];  // matrix (64 h + m) by rank
  __shared__ int16_t count_mem[kP4Waves][G * 64];  // squaring count by matrix
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Groups fit in 32 bits: the host takes this kernel only for operands below 2 GiB.
  const int32_t full = static_cast<int32_t>(args.batch / 64);
  const int32_t batches = full / G;
  const int32_t units = static_cast<int32_t>(sort_units<T, Pair>(args.batch));
  const int32_t stride = static_cast<int32_t>(gridDim.x) * kP4Waves;
  int32_t q = static_cast<int32_t>(blockIdx.x) * kP4Waves + wave;
  const U32x4 xs = rsrc_words(args.x.data);
  const U32x4 gs = rsrc_words(Pair ? args.g.data : args.x.data);
  const __amdgpu_buffer_rsrc_t out_rs = make_rsrc(args.out, 0x7FFFFFFFu);
  uint8_t* order = order_mem[wave];
  int16_t* count = count_mem[wave];
  auto issue = [&](int32_t b, char* slot) {
    const uint32_t a = lds_address(slot);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      load_group_to_lds<T>(xs, a + h * Slot::kGroup, (G * b + h) * kGroupBytes, lane);
      if constexpr (Pair) load_group_to_lds<T>(gs, a + h * Slot::kGroup + Slot::kArea, (G * b + h) * kGroupBytes, lane);
    }
  };
  auto matrix_at = [&](const char* grp, int m) {
    PM<Pair> cur;
    cur.d = decode<T, XL>(read_tuples_at<T>(grp, m));
    if constexpr (Pair) cur.u = decode<T, GL>(read_tuples_at<T>(grp + Slot::kArea, m));
    return cur;
  };
  int which = 0;
  if (q < batches) issue(q, tile_mem[wave][0]);
  for (bool first = true; q < batches; q += stride, first = false) {
    char* slot = tile_mem[wave][which];
    if constexpr (Slot::kSlots == 2) {
      // The next batch's loads go to the other slot (its results were read
      // out for the previous batch's stores); then wait for this batch's.
      if (q + stride < batches) {
        issue(q + stride, tile_mem[wave][which ^ 1]);
        wait_vm<kLoads>();
      } else {
        wait_vm<0>();
      }
    } else {
      // One slot: a later batch of this wavefront loads once the previous
      // batch's results have been read out of the slot for its stores.
      if (!first) issue(q, slot);
      wait_vm<0>();
    }
    lds_order();
    // Squaring count of matrix `lane` of each group (-1: non-finite, squares as 0).
    int sh[G], kh[G], rh[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      sh[h] = lane_squarings<Pair>(matrix_at(slot + h * Slot::kGroup, lane));
      kh[h] = sh[h] < 0 ? 0 : sh[h];
      rh[h] = 0;
    }
    // Rank by (count, matrix): counting sort, one ballot per count value and group.
    int base = 0;
    for (int v = 0; base < G * 64; ++v) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const uint64_t b = __builtin_amdgcn_ballot_w64(kh[h] == v);
        if (kh[h] == v) rh[h] = base + lanes_below(b);
        base += __builtin_popcountll(b);
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      order[rh[h]] = static_cast<uint8_t>(64 * h + lane);
      count[64 * h + lane] = static_cast<int16_t>(sh[h]);  // at most ~130 for finite 2-byte inputs
      if (args.s_out) args.s_out[static_cast<int64_t>(G * q + h) * 64 + lane] = sh[h];
    }
    lds_order();
#pragma unroll 1
    for (int r = 0; r < G; ++r) {
      const int id = order[64 * r + lane];
      const int s = count[id];
      char* grp = slot + (id >> 6) * Slot::kGroup;
      const int m = id & 63;
      const PM<Pair> a = scaled<Pair>(matrix_at(grp, m), s, args.x.sign, args.g.sign);
      const bool nan_free = !any_lane(s > kNanFreeCount);
      squarings<Pair>(t18<Pair>(a), s, [&](const M4& out) { write_result_at<T>(grp, m, out, nan_free); });
      if (s < 0) {  // rare: overwrite the result with NaN
        M4 nan;
#pragma unroll
        for (int e = 0; e < 16; ++e) nan.v[e] = __builtin_nanf("");
        write_result_at<T>(grp, m, nan, true);
      }
    }
    lds_order();
    // Store instruction c of a group: lane l's tuple c, to tuple C l + c of the group's block.
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const uint4 v = *reinterpret_cast<const uint4*>(slot + h * Slot::kGroup + c * kDenseRowBytes + 16 * lane);
        const U32x4 w = {v.x, v.y, v.z, v.w};
        __builtin_amdgcn_raw_buffer_store_b128(w, out_rs, (G * q + h) * kGroupBytes + 16 * (C * lane + c),
                                               kStoreSOffset, kNontemporal);
      }
    lds_order();
    if constexpr (Slot::kSlots == 2) which ^= 1;
  }
  // The groups after the last batch (full ones, then the partial last group),
  // one per unit.
  for (; q < units; q += stride) expm_group_elements<T, Pair>(args, static_cast<int64_t>(batches) * G + (q - batches), lane);
}

// Every group of an element-class batch (n < 4 or strides no vector class
// fits): per-element loads and stores.
template <typename T, bool Pair>
__global__ __launch_bounds__(64 * kP4Waves) __attribute__((amdgpu_waves_per_eu(Pair ? 2 : 4, 8))) void expm_p4_elem_kernel(
    ExpmArgs args) {
  const int lane = threadIdx.x & 63;
  const int64_t groups = (args.batch + 63) / 64;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kP4Waves;
  for (int64_t group = static_cast<int64_t>(blockIdx.x) * kP4Waves + (threadIdx.x >> 6); group < groups;
       group += stride)
    expm_group_elements<T, Pair>(args, group, lane);
}

// Workgroups of a launch: one wavefront per work unit, at most `cap`; each
// wavefront walks the units with a grid stride.  Most launches pass the
// resident count (a persistent grid whose next-unit prefetch hides the loads);
// the dense forward kernels pass kForwardGridCap, so that each wavefront takes
// one unit and the hardware starts a workgroup as another retires: C2 forward
// 23.3 -> 22.0 us, C3 24.6 -> 22.9 us against the persistent grid (same
// process, alternating), where the Frechet kernels lost 3-4% the same way.
constexpr int64_t kForwardGridCap = int64_t{1} << 20;  // keeps grid x 256 threads below 2^32

template <typename K>
hipError_t launch_persistent(K kernel, int64_t groups, const ExpmArgs& args, hipStream_t stream, int64_t cap) {
  int64_t grid = (groups + kP4Waves - 1) / kP4Waves;
  if (grid > cap) grid = cap;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(64 * kP4Waves), 0, stream, args);
  return hipGetLastError();
}

template <typename T, bool Pair, int XL, int GL, bool XD, bool GD>
hipError_t launch_vec(const ExpmArgs& args, hipStream_t stream) {
  // Persistent grid: as many workgroups as the device keeps resident at once.
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_p4_kernel<T, Pair, XL, GL, XD, GD>), 64 * kP4Waves);
  // Full groups, plus the wavefront after them for a partial last group.
  const int64_t groups = args.batch / 64 + (args.batch % 64 != 0);
  return launch_persistent(expm_p4_kernel<T, Pair, XL, GL, XD, GD>, groups, args, stream, resident);
}

template <typename T, bool Pair, int XL, int GL>
hipError_t launch_dma(const ExpmArgs& args, hipStream_t stream) {
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_p4_dma_kernel<T, Pair, XL, GL>), 64 * kP4Waves);
  const int64_t groups = args.batch / 64 + (args.batch % 64 != 0);
  return launch_persistent(expm_p4_dma_kernel<T, Pair, XL, GL>, groups, args, stream,
                           Pair ? resident : kForwardGridCap);
}

template <typename T, bool Pair, int XL, int GL>
hipError_t launch_sort(const ExpmArgs& args, hipStream_t stream) {
  static const int64_t resident =
      resident_blocks(reinterpret_cast<const void*>(&expm_p4_sort_kernel<T, Pair, XL, GL>), 64 * kP4Waves);
  // Batches of G full groups, then one unit per left-over group.
  return launch_persistent(expm_p4_sort_kernel<T, Pair, XL, GL>, sort_units<T, Pair>(args.batch), args, stream,
                           Pair ? resident : kForwardGridCap);
}

template <typename T, bool Pair, int XL, int GL>
hipError_t launch_vec_dense(const ExpmArgs& args, hipStream_t stream) {
  const bool xd = args.x.dense != 0;
  const bool gd = Pair && args.g.dense != 0;
  if (xd && (!Pair || gd)) {
    if constexpr (sizeof(typename T::storage) == 2) {
      return launch_sort<T, Pair, XL, GL>(args, stream);
    } else {
      return launch_dma<T, Pair, XL, GL>(args, stream);
    }
  }
  if (xd) {
    if constexpr (Pair) {
      return gd ? launch_vec<T, Pair, XL, GL, true, true>(args, stream)
                : launch_vec<T, Pair, XL, GL, true, false>(args, stream);
    } else {
      return launch_vec<T, Pair, XL, GL, true, false>(args, stream);
    }
  }
  if constexpr (Pair) {
    if (gd) return launch_vec<T, Pair, XL, GL, false, true>(args, stream);
  }
  return launch_vec<T, Pair, XL, GL, false, false>(args, stream);
}

// The vector classes address an operand through a buffer resource with 32-bit
// offsets: every byte a group touches must lie below 2^31 with non-negative
// strides; otherwise the element kernel (64-bit indexing) runs.
bool vec_addressable(const Operand& op, int64_t batch, int es) {
  constexpr int64_t kLimit = (int64_t{1} << 31) - 1024;
  if (op.sb < 0 || op.sr < 0 || op.sc < 0 || op.sr > kLimit || op.sc > kLimit) return false;
  const int64_t groups = (batch + 63) / 64;
  int64_t last = 0;  // any overflow means far beyond the 32-bit offsets
  if (__builtin_mul_overflow(groups * 64 - 1, op.sb, &last)) return false;
  last += 3 * (op.sr + op.sc) + 4;
  return last < kLimit / es;
}

template <typename T, bool Pair>
hipError_t launch_p4_t(const ExpmArgs& args, hipStream_t stream) {
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  int xl = args.n == 4 ? args.x.vec : kVecNone;
  int gl = (Pair && args.n == 4) ? args.g.vec : kVecNone;
  const bool addressable = vec_addressable(args.x, args.batch, es) && (!Pair || vec_addressable(args.g, args.batch, es)) &&
                           args.batch < ((int64_t{1} << 31) - 1024) / (16 * es);
  if (xl == kVecNone || (Pair && gl == kVecNone) || !addressable) {
    static const int64_t resident =
        resident_blocks(reinterpret_cast<const void*>(&expm_p4_elem_kernel<T, Pair>), 64 * kP4Waves);
    return launch_persistent(expm_p4_elem_kernel<T, Pair>, (args.batch + 63) / 64, args, stream, resident);
  }
  if constexpr (Pair) {
    if (xl == kVecRows) {
      return gl == kVecRows ? launch_vec_dense<T, Pair, kVecRows, kVecRows>(args, stream)
                            : launch_vec_dense<T, Pair, kVecRows, kVecCols>(args, stream);
    }
    return gl == kVecRows ? launch_vec_dense<T, Pair, kVecCols, kVecRows>(args, stream)
                          : launch_vec_dense<T, Pair, kVecCols, kVecCols>(args, stream);
  } else {
    return xl == kVecRows ? launch_vec_dense<T, Pair, kVecRows, kVecNone>(args, stream)
                          : launch_vec_dense<T, Pair, kVecCols, kVecNone>(args, stream);
  }
}

}  // namespace

hipError_t launch_p4(const ExpmArgs& args, int dtype, bool pair, hipStream_t stream) {
  if (dtype == F32::code) return pair ? launch_p4_t<F32, true>(args, stream) : launch_p4_t<F32, false>(args, stream);
  if (dtype == BF16::code) return pair ? launch_p4_t<BF16, true>(args, stream) : launch_p4_t<BF16, false>(args, stream);
  return pair ? launch_p4_t<F16, true>(args, stream) : launch_p4_t<F16, false>(args, stream);
}

}  // namespace fh

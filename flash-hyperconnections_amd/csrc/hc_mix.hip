// Hyper-connection stream mixing with the exponential fused in:
//   forward   Y_b = exp(H_b) X_b                         H [B, n, n], X [B, n, C]
//   backward  dX_b = exp(H_b)^T dY_b,
//             dE_b = dY_b X_b^T,  dH_b = L(H_b^T, dE_b)   (the gradient of exp)
// for n = 2..4 residual streams and any width C.  Nothing of the reference
// fuses this; its matrix_exp (ops/matrix_exp/__init__.py:80-97) returns
// exp(H) to the caller, who multiplies.  Here exp(H_b) never leaves the chip:
//
// * A wavefront takes a set of kTokens tokens spread over the batch: set k of
//   S = ceil(B / kTokens) holds tokens k, k + S, k + 2S, ..., so wavefronts
//   running at the same time stream neighbouring tokens and the rows in flight
//   form one contiguous region of HBM (consecutive tokens per wavefront put
//   every concurrent access 8 tokens apart, a power-of-two stride that costs
//   about 15% of the bandwidth).  Lane l computes exp(H) of the set's token
//   l % kTokens with the per-lane P == 4 code (p4_lane.h, the same arithmetic
//   as the matrix-exponential kernel, so E is bit-identical to it) and parks
//   it in the wavefront's LDS.
// * The wavefront then streams each token's rows: every lane loads 16 bytes
//   of each of the n rows per chunk (the whole wavefront covers 1 KB of each
//   row per chunk, coalesced), multiplies by E read back from LDS (one
//   broadcast read per token) and stores 16 bytes of each output row.  Rows
//   are read and written once, with the nontemporal cache hint.  Rows
//   are addressed through a buffer resource rebased per token in SGPRs, so no
//   VALU address arithmetic is needed and offsets never exceed one token.
// * The backward accumulates dE_b = dY_b X_b^T per lane over its columns (in
//   column order), reduces the 16 partial sums across the wavefront with a
//   fixed exchange tree (the result does not depend on anything but the
//   data), parks dE_b in LDS, and after its tokens each lane runs the P == 4
//   Frechet polynomial on (H^T, dE) of one token -- the same arithmetic as the
//   Frechet kernel.
//
// Both directions are bound by HBM traffic (16 FMAs per 2n elements moved
// forward, 32 per 3n backward); the exponential and Frechet work per token is
// small beside C >= a few hundred columns.
#include "p4_lane.h"

namespace fh {
namespace {

using namespace p4;

constexpr int kWaves = 4;   // wavefronts per workgroup
constexpr int kTokens = 8;  // tokens per wavefront

struct HcArgs {
  Operand h;        // [B, n, n]
  const void* x;    // [B, n, C], unit column stride
  int64_t xb, xr;   // element strides of X (token, row)
  const void* gy;   // backward: dY [B, n, C], unit column stride
  int64_t gb, gr;
  void* out;        // forward: Y, backward: dX; contiguous [B, n, C]
  void* dh;         // backward: dH, contiguous [B, n, n]
  float* aux;       // optional FP32 [B, n, n]: exp(H) (forward) or dE (backward)
  int64_t batch;
  int64_t cols;
  int n;
};

// Buffer resource over `bytes` bytes at `base` + `offset_elems` elements (uniform).
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rebased(const void* base, int64_t offset_elems, int64_t bytes) {
  const char* p = static_cast<const char*>(base) + offset_elems * static_cast<int64_t>(sizeof(typename T::storage));
  return make_rsrc(p, static_cast<uint32_t>(bytes));
}

// 16 bytes of storage as FP32 values (4 for FP32, 8 for FP16/BF16).
template <typename T>
struct Vec {
  static constexpr int V = 16 / static_cast<int>(sizeof(typename T::storage));
  float f[V];
};

template <typename T>
__device__ __forceinline__ Vec<T> unpack(U32x4 w) {
  using S = typename T::storage;
  Vec<T> r;
#pragma unroll
  for (int i = 0; i < Vec<T>::V; ++i) {
    if constexpr (sizeof(S) == 4) {
      r.f[i] = __uint_as_float(w[i]);
    } else {
      const uint16_t h = static_cast<uint16_t>(w[i >> 1] >> (16 * (i & 1)));
      r.f[i] = to_f32<T>(__builtin_bit_cast(S, h));
    }
  }
  return r;
}

template <typename T>
__device__ __forceinline__ U32x4 pack(const Vec<T>& v) {
  using S = typename T::storage;
  U32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (sizeof(S) == 4) {
      w[i] = __float_as_uint(v.f[i]);
    } else {
      w[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v.f[2 * i]))) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v.f[2 * i + 1]))) << 16);
    }
  }
  return w;
}

// Stream rows with the nontemporal hint (cache-policy bit 1: "nt" on gfx950).
constexpr int kStreamPolicy = 2;

__device__ __forceinline__ U32x4 load16(__amdgpu_buffer_rsrc_t rs, int32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, kStreamPolicy);
}

__device__ __forceinline__ void store16(U32x4 w, __amdgpu_buffer_rsrc_t rs, int32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b128(w, rs, voff, 0, kStreamPolicy);
}

// Token set `k` of `sets` = ceil(batch / kTokens): tokens k + i * sets, i < count.
struct TokenSet {
  int64_t first, stride;
  int count;
  __device__ __forceinline__ int64_t token(int i) const { return first + i * stride; }
};

__device__ __forceinline__ TokenSet token_set(int64_t k, int64_t sets, int64_t batch) {
  const int64_t left = (batch - k + sets - 1) / sets;
  return TokenSet{k, sets, static_cast<int>(left < kTokens ? left : kTokens)};
}

// exp(H) of token `b` for this lane (valid lanes), NaN for a non-finite H
// (csrc/MatrixExpSmall.cuh:126-140).
template <typename T, int N>
__device__ __forceinline__ M4 exp_of_token(const Operand& h, int64_t b, bool valid) {
  PM<false> cur;
  if (valid) {
    cur.d = load_elements<T>(h, b, N);
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) cur.d.v[e] = 0.f;
  }
  M4 e;
  const int s = expm_lane<false>(cur, h.sign, 1.f, [&](const M4& out) { e = out; });
  if (s < 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) e.v[i] = __builtin_nanf("");
  }
  return e;
}

// The wavefront's token set: lane l holds exp(H) of token l % kTokens of the
// set and lanes below kTokens park it in `etile` (16 floats per token); `aux`
// (optional) receives it in FP32.
template <typename T, int N>
__device__ __forceinline__ void exp_tokens(const HcArgs& a, const TokenSet& ts, int lane, float* etile) {
  const int slot = lane & (kTokens - 1);
  const int64_t b = ts.token(slot);
  const bool valid = slot < ts.count;
  const M4 e = exp_of_token<T, N>(a.h, b, valid);
  if (lane < kTokens) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<float4*>(etile + 16 * lane + 4 * q) =
          make_float4(e.v[4 * q], e.v[4 * q + 1], e.v[4 * q + 2], e.v[4 * q + 3]);
    if (a.aux && valid) {
#pragma unroll
      for (int i = 0; i < N; ++i)
#pragma unroll
        for (int j = 0; j < N; ++j) a.aux[b * N * N + i * N + j] = e.v[4 * i + j];
    }
  }
  lds_order();
}

__device__ __forceinline__ M4 read_token(const float* tile, int i) {
  M4 m;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 v = *reinterpret_cast<const float4*>(tile + 16 * i + 4 * q);
    m.v[4 * q] = v.x;
    m.v[4 * q + 1] = v.y;
    m.v[4 * q + 2] = v.z;
    m.v[4 * q + 3] = v.w;
  }
  return m;
}

// 16-byte column chunks per lane in flight per token: the forward keeps four
// (n loads each); the backward, which loads X and dY, two -- so that it fits
// two wavefronts per SIMD beside the Frechet polynomial's registers.
constexpr int kChunks = 4;
constexpr int kChunksBwd = 2;

// Forward: Y_b = E_b X_b, row i of Y = sum_k E[i][k] X[k] (fmaf chain k = 0..n-1 from +0).
template <typename T, int N>
__global__ __launch_bounds__(64 * kWaves) void hc_mix_fwd_kernel(HcArgs a) {
  __shared__ __attribute__((aligned(16))) float etile_mem[kWaves][kTokens * 16];
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  constexpr int V = Vec<T>::V;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* etile = etile_mem[wave];
  const int64_t sets = (a.batch + kTokens - 1) / kTokens;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWaves;
  const int64_t span = static_cast<int64_t>(64) * V * kChunks;  // columns per pass
  for (int64_t set = static_cast<int64_t>(blockIdx.x) * kWaves + wave; set < sets; set += stride) {
    const TokenSet ts = token_set(set, sets, a.batch);
    exp_tokens<T, N>(a, ts, lane, etile);
    for (int i = 0; i < ts.count; ++i) {
      const int64_t b = ts.token(i);
      const M4 e = read_token(etile, i);
      const __amdgpu_buffer_rsrc_t xs = rebased<T>(a.x, b * a.xb, ((N - 1) * a.xr + a.cols) * es);
      const __amdgpu_buffer_rsrc_t ys = rebased<T>(a.out, b * N * a.cols, N * a.cols * es);
      for (int64_t c0 = 0; c0 < a.cols; c0 += span) {
        U32x4 raw[kChunks][N];
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
          const int64_t c = c0 + (u * 64 + lane) * V;
#pragma unroll
          for (int k = 0; k < N; ++k)
            raw[u][k] = c < a.cols ? load16(xs, static_cast<int32_t>((k * a.xr + c) * es)) : U32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
          const int64_t c = c0 + (u * 64 + lane) * V;
          Vec<T> xv[N];
#pragma unroll
          for (int k = 0; k < N; ++k) xv[k] = unpack<T>(raw[u][k]);
#pragma unroll
          for (int i2 = 0; i2 < N; ++i2) {
            Vec<T> y;
#pragma unroll
            for (int v = 0; v < V; ++v) {
              float acc = __builtin_fmaf(e.v[4 * i2], xv[0].f[v], 0.f);
#pragma unroll
              for (int k = 1; k < N; ++k) acc = __builtin_fmaf(e.v[4 * i2 + k], xv[k].f[v], acc);
              y.f[v] = acc;
            }
            if (c < a.cols) store16(pack<T>(y), ys, static_cast<int32_t>((i2 * a.cols + c) * es));
          }
        }
      }
    }
    lds_order();
  }
}

// Sum of 16 per-lane values over the wavefront, reduce-scatter style: after
// exchanging halves with the lane 1, 2, 4, 8 apart (keeping the half this
// lane's bit selects) every lane of a 16-lane row holds the row's sum of one
// entry, entry = bit-reverse(lane & 15); two more exchanges (16, 32 apart) add
// the rows.  Fixed order: every entry's sum is ((r0 + r1) + (r2 + r3)) of
// fixed per-row trees.  Returns the total of entry bitrev4(lane & 15).
__device__ __forceinline__ float wave_sum16(const float (&v)[16], int lane) {
  float a[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) a[e] = v[e];
#pragma unroll
  for (int step = 0; step < 4; ++step) {
    const int half = 8 >> step;
    const bool upper = (lane >> step) & 1;
#pragma unroll
    for (int j = 0; j < half; ++j) {
      const float keep = upper ? a[j + half] : a[j];
      const float send = upper ? a[j] : a[j + half];
      a[j] = keep + __shfl_xor(send, 1 << step);
    }
  }
  float t = a[0] + __shfl_xor(a[0], 16);
  return t + __shfl_xor(t, 32);
}

__device__ __forceinline__ int bitrev4(int x) { return ((x & 1) << 3) | ((x & 2) << 1) | ((x & 4) >> 1) | ((x & 8) >> 3); }

// Backward: dX row k = sum_r E[r][k] dY[r] (fmaf chain r = 0..n-1 from +0);
// dE[r][k] = sum_c dY[r][c] X[k][c] (per lane in column order, then
// wave_sum16); dH = L(H^T, dE).
template <typename T, int N>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 8))) void hc_mix_bwd_kernel(HcArgs a) {
  __shared__ __attribute__((aligned(16))) float etile_mem[kWaves][kTokens * 16];
  __shared__ __attribute__((aligned(16))) float gtile_mem[kWaves][kTokens * 16];
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  constexpr int V = Vec<T>::V;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* etile = etile_mem[wave];
  float* gtile = gtile_mem[wave];
  const int64_t sets = (a.batch + kTokens - 1) / kTokens;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWaves;
  const int64_t span = static_cast<int64_t>(64) * V * kChunksBwd;
  for (int64_t set = static_cast<int64_t>(blockIdx.x) * kWaves + wave; set < sets; set += stride) {
    const TokenSet ts = token_set(set, sets, a.batch);
    exp_tokens<T, N>(a, ts, lane, etile);
    for (int i = 0; i < ts.count; ++i) {
      const int64_t b = ts.token(i);
      const M4 e = read_token(etile, i);
      const __amdgpu_buffer_rsrc_t xs = rebased<T>(a.x, b * a.xb, ((N - 1) * a.xr + a.cols) * es);
      const __amdgpu_buffer_rsrc_t gs = rebased<T>(a.gy, b * a.gb, ((N - 1) * a.gr + a.cols) * es);
      const __amdgpu_buffer_rsrc_t ds = rebased<T>(a.out, b * N * a.cols, N * a.cols * es);
      float acc[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[q] = 0.f;
      for (int64_t c0 = 0; c0 < a.cols; c0 += span) {
        U32x4 xr[kChunksBwd][N], gr[kChunksBwd][N];
#pragma unroll
        for (int u = 0; u < kChunksBwd; ++u) {
          const int64_t c = c0 + (u * 64 + lane) * V;
#pragma unroll
          for (int k = 0; k < N; ++k) {
            xr[u][k] = c < a.cols ? load16(xs, static_cast<int32_t>((k * a.xr + c) * es)) : U32x4{0, 0, 0, 0};
            gr[u][k] = c < a.cols ? load16(gs, static_cast<int32_t>((k * a.gr + c) * es)) : U32x4{0, 0, 0, 0};
          }
        }
#pragma unroll
        for (int u = 0; u < kChunksBwd; ++u) {
          const int64_t c = c0 + (u * 64 + lane) * V;
          Vec<T> xv[N], gv[N];
#pragma unroll
          for (int k = 0; k < N; ++k) {
            xv[k] = unpack<T>(xr[u][k]);
            gv[k] = unpack<T>(gr[u][k]);
          }
#pragma unroll
          for (int k = 0; k < N; ++k) {
            Vec<T> dx;
#pragma unroll
            for (int v = 0; v < V; ++v) {
              float d = __builtin_fmaf(e.v[k], gv[0].f[v], 0.f);
#pragma unroll
              for (int r = 1; r < N; ++r) d = __builtin_fmaf(e.v[4 * r + k], gv[r].f[v], d);
              dx.f[v] = d;
            }
            if (c < a.cols) store16(pack<T>(dx), ds, static_cast<int32_t>((k * a.cols + c) * es));
          }
#pragma unroll
          for (int r = 0; r < N; ++r)
#pragma unroll
            for (int k = 0; k < N; ++k)
#pragma unroll
              for (int v = 0; v < V; ++v) acc[4 * r + k] = __builtin_fmaf(gv[r].f[v], xv[k].f[v], acc[4 * r + k]);
        }
      }
      const float total = wave_sum16(acc, lane);
      if (lane < 16) gtile[16 * i + bitrev4(lane)] = total;
    }
    lds_order();
    // L(H^T, dE) of the set's token lane % kTokens.
    const int slot = lane & (kTokens - 1);
    const int64_t b = ts.token(slot);
    const bool valid = slot < ts.count;
    PM<true> cur;
    if (valid) {
      const M4 h = load_elements<T>(a.h, b, N);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) cur.d.v[4 * r + c] = h.v[4 * c + r];
      cur.u = read_token(gtile, slot);
      // The debug copy of dE goes out now, so that cur.u is not kept live
      // across the Frechet polynomial (it would spill at the 256-VGPR cap).
      if (a.aux && lane < kTokens) {
#pragma unroll
        for (int r = 0; r < N; ++r)
#pragma unroll
          for (int k = 0; k < N; ++k) a.aux[b * N * N + r * N + k] = cur.u.v[4 * r + k];
      }
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        cur.d.v[q] = 0.f;
        cur.u.v[q] = 0.f;
      }
    }
    M4 dh;
    const int s = expm_lane<true>(cur, a.h.sign, 1.f, [&](const M4& out) { dh = out; });
    if (s < 0) {
#pragma unroll
      for (int q = 0; q < 16; ++q) dh.v[q] = __builtin_nanf("");
    }
    if (lane < kTokens && valid) store_elements<T>(a.dh, b, N, dh);
    lds_order();
  }
}

// ---- 5 <= n <= 8 streams: exp(H) supplied in FP32 ----------------------------
//
// For n = 5..8 the exponential runs in its own kernel (P = 8, FP32 output, the
// same bits the fused path would keep on chip); these kernels apply it.  The
// token sets, row streaming and nontemporal hints are the fused kernels'.
// E of the set's tokens sits in LDS in rows of 8 floats (64 per token): E
// itself for the forward, E^T for the backward, so that the row an output
// row needs is two 16-byte broadcast reads.

struct WideArgs {
  const float* e;   // FP32 [B, n, n], contiguous
  const void* x;    // [B, n, C], unit column stride
  int64_t xb, xr;
  const void* gy;   // backward: dY [B, n, C], unit column stride
  int64_t gb, gr;
  void* out;        // forward: Y, backward: dX; contiguous [B, n, C]
  float* de;        // backward: dE = dY X^T, FP32 [B, n, n], contiguous
  int64_t batch;
  int64_t cols;
  int n;
};

constexpr int kWideChunks = 2;     // 16-byte column chunks per lane in flight (forward)
constexpr int kWideChunksBwd = 2;  // 8-byte column chunks per lane in flight (backward)

// 8 bytes of storage as FP32 values (2 for FP32, 4 for FP16/BF16).
template <typename T>
struct Vec8 {
  static constexpr int V = 8 / static_cast<int>(sizeof(typename T::storage));
  float f[V];
};

template <typename T>
__device__ __forceinline__ Vec8<T> unpack8(U32x2 w) {
  using S = typename T::storage;
  Vec8<T> r;
#pragma unroll
  for (int i = 0; i < Vec8<T>::V; ++i) {
    if constexpr (sizeof(S) == 4) {
      r.f[i] = __uint_as_float(w[i]);
    } else {
      const uint16_t h = static_cast<uint16_t>(w[i >> 1] >> (16 * (i & 1)));
      r.f[i] = to_f32<T>(__builtin_bit_cast(S, h));
    }
  }
  return r;
}

template <typename T>
__device__ __forceinline__ U32x2 pack8(const Vec8<T>& v) {
  using S = typename T::storage;
  U32x2 w;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if constexpr (sizeof(S) == 4) {
      w[i] = __float_as_uint(v.f[i]);
    } else {
      w[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v.f[2 * i]))) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v.f[2 * i + 1]))) << 16);
    }
  }
  return w;
}

__device__ __forceinline__ U32x2 load8(__amdgpu_buffer_rsrc_t rs, int32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b64(rs, voff, 0, kStreamPolicy);
}

__device__ __forceinline__ void store8(U32x2 w, __amdgpu_buffer_rsrc_t rs, int32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b64(w, rs, voff, 0, kStreamPolicy);
}

// E of the set's tokens into `etile` (64 floats per token, rows of 8): lane
// 8 j + p copies row p of token j's E (transposed: column p) when both exist.
template <int N, bool Transposed>
__device__ __forceinline__ void load_set_e(const WideArgs& a, const TokenSet& ts, int lane, float* etile) {
  const int j = lane >> 3;
  const int p = lane & 7;
  if (j < ts.count && p < N) {
    const float* src = a.e + ts.token(j) * (N * N);
#pragma unroll
    for (int k = 0; k < N; ++k) etile[64 * j + 8 * p + k] = Transposed ? src[k * N + p] : src[p * N + k];
  }
  lds_order();
}

// Row r of the token's 8-float rows (the first N entries are used).
__device__ __forceinline__ void read_row8(const float* tile, int token, int r, float (&row)[8]) {
  const float4 lo = *reinterpret_cast<const float4*>(tile + 64 * token + 8 * r);
  const float4 hi = *reinterpret_cast<const float4*>(tile + 64 * token + 8 * r + 4);
  row[0] = lo.x; row[1] = lo.y; row[2] = lo.z; row[3] = lo.w;
  row[4] = hi.x; row[5] = hi.y; row[6] = hi.z; row[7] = hi.w;
}

// Forward: row i of Y = sum_k E[i][k] X[k] (fmaf chain k = 0..n-1 from +0).
template <typename T, int N>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 8))) void hc_wide_fwd_kernel(WideArgs a) {
  __shared__ __attribute__((aligned(16))) float etile_mem[kWaves][kTokens * 64];
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  constexpr int V = Vec<T>::V;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* etile = etile_mem[wave];
  const int64_t sets = (a.batch + kTokens - 1) / kTokens;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWaves;
  const int64_t span = static_cast<int64_t>(64) * V * kWideChunks;
  for (int64_t set = static_cast<int64_t>(blockIdx.x) * kWaves + wave; set < sets; set += stride) {
    const TokenSet ts = token_set(set, sets, a.batch);
    load_set_e<N, false>(a, ts, lane, etile);
    for (int i = 0; i < ts.count; ++i) {
      const int64_t b = ts.token(i);
      float e[N][8];
#pragma unroll
      for (int r = 0; r < N; ++r) read_row8(etile, i, r, e[r]);
      const __amdgpu_buffer_rsrc_t xs = rebased<T>(a.x, b * a.xb, ((N - 1) * a.xr + a.cols) * es);
      const __amdgpu_buffer_rsrc_t ys = rebased<T>(a.out, b * N * a.cols, N * a.cols * es);
      for (int64_t c0 = 0; c0 < a.cols; c0 += span) {
        U32x4 raw[kWideChunks][N];
#pragma unroll
        for (int u = 0; u < kWideChunks; ++u) {
          const int64_t c = c0 + (u * 64 + lane) * V;
#pragma unroll
          for (int k = 0; k < N; ++k)
            raw[u][k] = c < a.cols ? load16(xs, static_cast<int32_t>((k * a.xr + c) * es)) : U32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kWideChunks; ++u) {
          const int64_t c = c0 + (u * 64 + lane) * V;
          Vec<T> xv[N];
#pragma unroll
          for (int k = 0; k < N; ++k) xv[k] = unpack<T>(raw[u][k]);
#pragma unroll
          for (int i2 = 0; i2 < N; ++i2) {
            Vec<T> y;
#pragma unroll
            for (int v = 0; v < V; ++v) {
              float acc = __builtin_fmaf(e[i2][0], xv[0].f[v], 0.f);
#pragma unroll
              for (int k = 1; k < N; ++k) acc = __builtin_fmaf(e[i2][k], xv[k].f[v], acc);
              y.f[v] = acc;
            }
            if (c < a.cols) store16(pack<T>(y), ys, static_cast<int32_t>((i2 * a.cols + c) * es));
          }
        }
      }
    }
    lds_order();
  }
}

// Sum of 64 per-lane values over the wavefront, reduce-scatter style: six
// exchanges with the lane 1, 2, 4, 8, 16, 32 apart, each keeping the half
// this lane's bit selects, leave every lane with the total of one entry,
// entry = bit-reverse(lane) (6 bits), summed in a fixed tree.
__device__ __forceinline__ float wave_sum64(const float (&v)[64], int lane) {
  float a[64];
#pragma unroll
  for (int e = 0; e < 64; ++e) a[e] = v[e];
#pragma unroll
  for (int step = 0; step < 6; ++step) {
    const int half = 32 >> step;
    const bool upper = (lane >> step) & 1;
#pragma unroll
    for (int j = 0; j < half; ++j) {
      const float keep = upper ? a[j + half] : a[j];
      const float send = upper ? a[j] : a[j + half];
      a[j] = keep + __shfl_xor(send, 1 << step);
    }
  }
  return a[0];
}

__device__ __forceinline__ int bitrev6(int x) {
  return ((x & 1) << 5) | ((x & 2) << 3) | ((x & 4) << 1) | ((x & 8) >> 1) | ((x & 16) >> 3) | ((x & 32) >> 5);
}

// Backward: dX row k = sum_r E[r][k] dY[r] (fmaf chain r = 0..n-1 from +0);
// dE[r][k] = sum_c dY[r][c] X[k][c] (per lane in column order, then
// wave_sum64), written to a.de.
template <typename T, int N>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 8))) void hc_wide_bwd_kernel(WideArgs a) {
  __shared__ __attribute__((aligned(16))) float etile_mem[kWaves][kTokens * 64];
  constexpr int es = static_cast<int>(sizeof(typename T::storage));
  constexpr int V = Vec8<T>::V;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* etile = etile_mem[wave];
  const int64_t sets = (a.batch + kTokens - 1) / kTokens;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kWaves;
  const int64_t span = static_cast<int64_t>(64) * V * kWideChunksBwd;
  const int entry = bitrev6(lane);
  for (int64_t set = static_cast<int64_t>(blockIdx.x) * kWaves + wave; set < sets; set += stride) {
    const TokenSet ts = token_set(set, sets, a.batch);
    load_set_e<N, true>(a, ts, lane, etile);
    for (int i = 0; i < ts.count; ++i) {
      const int64_t b = ts.token(i);
      const __amdgpu_buffer_rsrc_t xs = rebased<T>(a.x, b * a.xb, ((N - 1) * a.xr + a.cols) * es);
      const __amdgpu_buffer_rsrc_t gs = rebased<T>(a.gy, b * a.gb, ((N - 1) * a.gr + a.cols) * es);
      const __amdgpu_buffer_rsrc_t ds = rebased<T>(a.out, b * N * a.cols, N * a.cols * es);
      float acc[64];
#pragma unroll
      for (int q = 0; q < 64; ++q) acc[q] = 0.f;
      for (int64_t c0 = 0; c0 < a.cols; c0 += span) {
        U32x2 xr[kWideChunksBwd][N], gr[kWideChunksBwd][N];
#pragma unroll
        for (int u = 0; u < kWideChunksBwd; ++u) {
          const int64_t c = c0 + (u * 64 + lane) * V;
#pragma unroll
          for (int k = 0; k < N; ++k) {
            xr[u][k] = c < a.cols ? load8(xs, static_cast<int32_t>((k * a.xr + c) * es)) : U32x2{0, 0};
            gr[u][k] = c < a.cols ? load8(gs, static_cast<int32_t>((k * a.gr + c) * es)) : U32x2{0, 0};
          }
        }
#pragma unroll
        for (int u = 0; u < kWideChunksBwd; ++u) {
          const int64_t c = c0 + (u * 64 + lane) * V;
          Vec8<T> xv[N], gv[N];
#pragma unroll
          for (int k = 0; k < N; ++k) {
            xv[k] = unpack8<T>(xr[u][k]);
            gv[k] = unpack8<T>(gr[u][k]);
          }
#pragma unroll
          for (int k = 0; k < N; ++k) {
            float col[8];
            read_row8(etile, i, k, col);  // column k of E
            Vec8<T> dx;
#pragma unroll
            for (int v = 0; v < V; ++v) {
              float d = __builtin_fmaf(col[0], gv[0].f[v], 0.f);
#pragma unroll
              for (int r = 1; r < N; ++r) d = __builtin_fmaf(col[r], gv[r].f[v], d);
              dx.f[v] = d;
            }
            if (c < a.cols) store8(pack8<T>(dx), ds, static_cast<int32_t>((k * a.cols + c) * es));
          }
#pragma unroll
          for (int r = 0; r < N; ++r)
#pragma unroll
            for (int k = 0; k < N; ++k)
#pragma unroll
              for (int v = 0; v < V; ++v) acc[r * N + k] = __builtin_fmaf(gv[r].f[v], xv[k].f[v], acc[r * N + k]);
        }
      }
      const float total = wave_sum64(acc, lane);
      if (entry < N * N) a.de[b * (N * N) + entry] = total;
    }
    lds_order();
  }
}

// Grid: one wavefront per token set up to what the device keeps resident
// (counted once per kernel; the wavefronts stride over the rest).
template <typename T, int N, bool Backward>
hipError_t launch_one(const HcArgs& a, hipStream_t stream) {
  const auto kernel = Backward ? hc_mix_bwd_kernel<T, N> : hc_mix_fwd_kernel<T, N>;
  static const int64_t resident = resident_blocks(reinterpret_cast<const void*>(kernel), 64 * kWaves);
  const int64_t sets = (a.batch + kTokens - 1) / kTokens;
  int64_t grid = (sets + kWaves - 1) / kWaves;
  if (grid > resident) grid = resident;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), 0, stream, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const HcArgs& a, bool backward, hipStream_t stream) {
  switch (a.n) {
    case 2:
      return backward ? launch_one<T, 2, true>(a, stream) : launch_one<T, 2, false>(a, stream);
    case 3:
      return backward ? launch_one<T, 3, true>(a, stream) : launch_one<T, 3, false>(a, stream);
    default:
      return backward ? launch_one<T, 4, true>(a, stream) : launch_one<T, 4, false>(a, stream);
  }
}

template <typename T, int N, bool Backward>
hipError_t launch_wide_one(const WideArgs& a, hipStream_t stream) {
  const auto kernel = Backward ? hc_wide_bwd_kernel<T, N> : hc_wide_fwd_kernel<T, N>;
  static const int64_t resident = resident_blocks(reinterpret_cast<const void*>(kernel), 64 * kWaves);
  const int64_t sets = (a.batch + kTokens - 1) / kTokens;
  int64_t grid = (sets + kWaves - 1) / kWaves;
  if (grid > resident) grid = resident;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), 0, stream, a);
  return hipGetLastError();
}

template <typename T, bool Backward>
hipError_t launch_wide_t(const WideArgs& a, hipStream_t stream) {
  switch (a.n) {
    case 5:
      return launch_wide_one<T, 5, Backward>(a, stream);
    case 6:
      return launch_wide_one<T, 6, Backward>(a, stream);
    case 7:
      return launch_wide_one<T, 7, Backward>(a, stream);
    default:
      return launch_wide_one<T, 8, Backward>(a, stream);
  }
}

}  // namespace

hipError_t launch_hc_apply(const float* e, const void* x, const int64_t* xs, const void* gy, const int64_t* gs,
                           void* out, float* de, int dtype, int64_t batch, int n, int64_t cols, hipStream_t stream) {
  WideArgs a;
  a.e = e;
  a.x = x;
  a.xb = xs[0];
  a.xr = xs[1];
  a.gy = gy;
  a.gb = gs ? gs[0] : 0;
  a.gr = gs ? gs[1] : 0;
  a.out = out;
  a.de = de;
  a.batch = batch;
  a.cols = cols;
  a.n = n;
  if (gy != nullptr) {
    if (dtype == F32::code) return launch_wide_t<F32, true>(a, stream);
    if (dtype == BF16::code) return launch_wide_t<BF16, true>(a, stream);
    return launch_wide_t<F16, true>(a, stream);
  }
  if (dtype == F32::code) return launch_wide_t<F32, false>(a, stream);
  if (dtype == BF16::code) return launch_wide_t<BF16, false>(a, stream);
  return launch_wide_t<F16, false>(a, stream);
}

hipError_t launch_hc_mix(const Operand& h, const void* x, const int64_t* xs, const void* gy, const int64_t* gs,
                         void* out, void* dh, float* aux, int dtype, int64_t batch, int n, int64_t cols,
                         hipStream_t stream) {
  HcArgs a;
  a.h = h;
  a.x = x;
  a.xb = xs[0];
  a.xr = xs[1];
  a.gy = gy;
  a.gb = gs ? gs[0] : 0;
  a.gr = gs ? gs[1] : 0;
  a.out = out;
  a.dh = dh;
  a.aux = aux;
  a.batch = batch;
  a.cols = cols;
  a.n = n;
  const bool backward = gy != nullptr;
  if (dtype == F32::code) return launch_t<F32>(a, backward, stream);
  if (dtype == BF16::code) return launch_t<BF16>(a, backward, stream);
  return launch_t<F16>(a, backward, stream);
}

}  // namespace fh

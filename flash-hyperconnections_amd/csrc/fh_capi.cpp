// C-ABI entry points of libflash_hypercons_hip.so (declared in
// include/flash_hypercons.h): argument validation, operand description and
// kernel selection.  Replaces the reference's host launcher
// csrc/matrix_exp.cu:13-86 without its FP32/contiguous/padded staging copies:
// the kernels read the caller's strided storage directly and write only the
// logical n x n block.
#include <string>

#include "fh_kernels.h"
#include "flash_hypercons.h"

namespace {

thread_local std::string g_error;

// The reference's input check message (csrc/matrix_exp.cu:52-55).
constexpr const char* kInputMessage =
    "expected a strided CUDA [B, N, N] tensor, 2 <= N <= 32, in float32, float16, or bfloat16";
constexpr const char* kDirectionMessage = "matrix exponential direction must match the input";

int fail(int code, const std::string& message) {
  g_error = message;
  return code;
}

int element_size(int dtype) { return dtype == FH_DTYPE_F32 ? 4 : 2; }

bool aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

fh::Operand make_operand(const void* data, const int64_t strides[3], int neg, int dtype, int n) {
  fh::Operand op;
  op.data = data;
  op.sb = strides[0];
  op.sr = strides[1];
  op.sc = strides[2];
  op.sign = neg ? -1.f : 1.f;
  op.vec = fh::kVecNone;
  op.dense = 0;
  if (n == 4 || n == 8) {
    // Every row (or column) of the matrix is made of aligned 4-element
    // vectors when its elements are adjacent and every matrix/row (column)
    // start keeps the vector alignment; consecutive matrices are one
    // contiguous block (`dense`) when they are packed as well.
    const int64_t vbytes = 4 * element_size(dtype);
    const bool base_ok = aligned(data, vbytes) && strides[0] % 4 == 0;
    const bool packed = strides[0] == n * n && aligned(data, 16);
    if (base_ok && strides[2] == 1 && strides[1] % 4 == 0) {
      op.vec = fh::kVecRows;
      op.dense = packed && strides[1] == n;
    } else if (base_ok && strides[1] == 1 && strides[2] % 4 == 0) {
      op.vec = fh::kVecCols;
      op.dense = packed && strides[2] == n;
    }
  }
  return op;
}

// The P = 16/32 kernels address one matrix through a buffer resource with
// 32-bit offsets: its footprint ((n - 1) * (sr + sc) + 1 elements) must stay
// below 2 GiB and its strides non-negative.  Other operands go to the
// one-wavefront-per-matrix kernel, which indexes in 64 bits.
bool tile_addressable(const fh::Operand& op, int n, int dtype) {
  if (op.sr < 0 || op.sc < 0 || op.sb < 0) return false;
  const int64_t limit = (int64_t{1} << 31) - 1;
  const int64_t es = element_size(dtype);
  if (op.sr > limit || op.sc > limit) return false;
  return ((n - 1) * (op.sr + op.sc) + 1) * es <= limit;
}

int validate(const void* input, const int64_t* strides, int dtype, int64_t batch, int n, const void* out) {
  if (n < 2 || n > 32 || (dtype != FH_DTYPE_F32 && dtype != FH_DTYPE_BF16 && dtype != FH_DTYPE_F16) || batch < 0)
    return fail(FH_ERR_INVALID_ARGUMENT, kInputMessage);
  if (batch > 0 && (input == nullptr || strides == nullptr || out == nullptr))
    return fail(FH_ERR_INVALID_ARGUMENT, "null input, stride or output pointer");
  return FH_OK;
}

int launch(const void* input, const int64_t input_strides[3], int input_neg, const void* direction,
           const int64_t direction_strides[3], int direction_neg, void* out, int dtype, int64_t batch, int n,
           int variant, int32_t* s_out, hipStream_t stream) {
  int rc = validate(input, input_strides, dtype, batch, n, out);
  if (rc != FH_OK) return rc;
  if (variant != FH_VARIANT_AUTO && variant != FH_VARIANT_GENERIC)
    return fail(FH_ERR_INVALID_ARGUMENT, "unknown kernel variant");
  const bool pair = direction != nullptr;
  if (pair && batch > 0 && direction_strides == nullptr) return fail(FH_ERR_INVALID_ARGUMENT, kDirectionMessage);
  if (batch == 0) return FH_OK;  // csrc/matrix_exp.cu:62-64
  fh::ExpmArgs args;
  args.x = make_operand(input, input_strides, input_neg, dtype, n);
  if (pair) {
    args.g = make_operand(direction, direction_strides, direction_neg, dtype, n);
  } else {
    args.g = args.x;
  }
  args.out = out;
  args.s_out = s_out;
  args.batch = batch;
  args.n = n;
  const int P = n <= 4 ? 4 : n <= 8 ? 8 : n <= 16 ? 16 : 32;  // csrc/matrix_exp.cu:65
  hipError_t err;
  if (variant == FH_VARIANT_GENERIC) {
    err = fh::launch_generic(args, dtype, P, pair, stream);
  } else if (P == 4) {
    err = fh::launch_p4(args, dtype, pair, stream);
  } else if (P == 8) {
    err = fh::launch_oct(args, dtype, pair, stream);
  } else if (tile_addressable(args.x, n, dtype) && (!pair || tile_addressable(args.g, n, dtype))) {
    err = fh::launch_tile(args, dtype, P, pair, stream);
  } else {
    err = fh::launch_generic(args, dtype, P, pair, stream);
  }
  if (err != hipSuccess) return fail(FH_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(err));
  g_error.clear();
  return FH_OK;
}

// Operands of the fused stream mixing: H any strides; X (and dY) [B, n, C]
// with contiguous, 16-byte aligned rows of a whole number of 16-byte vectors,
// each token's rows spanning less than 2 GiB.
// Rows of a streamed operand ([B, n, C], unit column stride): 16-byte aligned,
// strides and C whole 16-byte vectors, each token's rows spanning < 2 GiB.
constexpr int64_t kSpan = int64_t{1} << 31;  // bytes one token's rows may span (32-bit buffer offsets)

// Layout the streaming kernels read in place: contiguous, 16-byte aligned rows
// whose length and strides are whole 16-byte vectors.
bool stream_rows_ok(const void* p, const int64_t* st, int64_t cols, int dtype) {
  const int64_t v = 16 / element_size(dtype);
  return st != nullptr && aligned(p, 16) && st[2] == 1 && st[0] >= 0 && st[1] >= 0 && st[0] % v == 0 &&
         st[1] % v == 0 && cols % v == 0;
}

// One token's n rows, read through row stride st[1], and the contiguous output
// token (n * cols elements) each span < 2 GiB: the kernels address a token
// through one buffer resource with 32-bit offsets.
bool stream_span_ok(const int64_t* st, int n, int64_t cols, int dtype) {
  const int64_t es = element_size(dtype);
  return st[1] < kSpan && cols < kSpan && ((n - 1) * st[1] + cols) * es < kSpan && n * cols * es < kSpan;
}

std::string span_message(const char* op) {
  return std::string(op) + ": one token's rows of X, dY and of the output must each span less than 2 GiB";
}

bool known_dtype(int dtype) { return dtype == FH_DTYPE_F32 || dtype == FH_DTYPE_BF16 || dtype == FH_DTYPE_F16; }

std::string rows_message(const char* op, int dtype) {
  return std::string(op) + ": X and dY need contiguous, 16-byte aligned rows whose length C and strides are multiples of " +
         std::to_string(16 / element_size(dtype)) + " elements";
}

int validate_hc(const void* h, const int64_t* hs, const void* x, const int64_t* xs, const void* g, const int64_t* gs,
                const void* out, int dtype, int64_t batch, int n, int64_t cols) {
  if (n < 2 || n > 4 || !known_dtype(dtype) || batch < 0 || cols < 1)
    return fail(FH_ERR_INVALID_ARGUMENT,
                "hc_mix: expected H [B, n, n] and X [B, n, C] with 2 <= n <= 4, C >= 1, in float32, float16, or "
                "bfloat16");
  if (batch == 0) return FH_OK;
  if (h == nullptr || hs == nullptr || x == nullptr || xs == nullptr || out == nullptr)
    return fail(FH_ERR_INVALID_ARGUMENT, "hc_mix: null pointer");
  if (!stream_rows_ok(x, xs, cols, dtype) || (g != nullptr && !stream_rows_ok(g, gs, cols, dtype)) ||
      !aligned(out, 16))
    return fail(FH_ERR_INVALID_ARGUMENT, rows_message("hc_mix", dtype));
  if (!stream_span_ok(xs, n, cols, dtype) || (g != nullptr && !stream_span_ok(gs, n, cols, dtype)))
    return fail(FH_ERR_INVALID_ARGUMENT, span_message("hc_mix"));
  return FH_OK;
}

// The apply entry points (5 <= n <= 8): E is FP32 [batch, n, n], contiguous.
int validate_apply(const float* e, const void* x, const int64_t* xs, const void* g, const int64_t* gs,
                   const void* out, int dtype, int64_t batch, int n, int64_t cols) {
  if (n < 5 || n > 8 || !known_dtype(dtype) || batch < 0 || cols < 1)
    return fail(FH_ERR_INVALID_ARGUMENT,
                "hc_apply: expected E [B, n, n] (float32) and X [B, n, C] with 5 <= n <= 8, C >= 1, in float32, "
                "float16, or bfloat16");
  if (batch == 0) return FH_OK;
  if (e == nullptr || x == nullptr || xs == nullptr || out == nullptr)
    return fail(FH_ERR_INVALID_ARGUMENT, "hc_apply: null pointer");
  if (!aligned(e, 4)) return fail(FH_ERR_INVALID_ARGUMENT, "hc_apply: E must be 4-byte aligned float32");
  if (!stream_rows_ok(x, xs, cols, dtype) || (g != nullptr && !stream_rows_ok(g, gs, cols, dtype)) ||
      !aligned(out, 16))
    return fail(FH_ERR_INVALID_ARGUMENT, rows_message("hc_apply", dtype));
  if (!stream_span_ok(xs, n, cols, dtype) || (g != nullptr && !stream_span_ok(gs, n, cols, dtype)))
    return fail(FH_ERR_INVALID_ARGUMENT, span_message("hc_apply"));
  return FH_OK;
}

}  // namespace

namespace fh {

Operand hc_operand(const void* h, const int64_t strides[3], int neg, int dtype) {
  return make_operand(h, strides, neg, dtype, 0);
}

int64_t resident_blocks(const void* kernel, int block) {
  int device = 0;
  int per_cu = 0;
  int cus = 0;
  if (hipGetDevice(&device) != hipSuccess) return 1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess) per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) cus = 1;
  const int64_t n = static_cast<int64_t>(per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
  return n > 0 ? n : 1;
}

}  // namespace fh

extern "C" {

int fh_matrix_exp(const void* input, const int64_t strides[3], int input_neg, void* out, int dtype, int64_t batch,
                  int n, hipStream_t stream) {
  return launch(input, strides, input_neg, nullptr, nullptr, 0, out, dtype, batch, n, FH_VARIANT_AUTO, nullptr,
                stream);
}

int fh_frechet(const void* input, const int64_t input_strides[3], int input_neg, const void* direction,
               const int64_t direction_strides[3], int direction_neg, void* out, int dtype, int64_t batch, int n,
               hipStream_t stream) {
  if (batch > 0 && direction == nullptr) return fail(FH_ERR_INVALID_ARGUMENT, kDirectionMessage);
  return launch(input, input_strides, input_neg, direction, direction_strides, direction_neg, out, dtype, batch, n,
                FH_VARIANT_AUTO, nullptr, stream);
}

int fh_expm_launch(const void* input, const int64_t input_strides[3], int input_neg, const void* direction,
                   const int64_t direction_strides[3], int direction_neg, void* out, int dtype, int64_t batch, int n,
                   int variant, int32_t* s_out, hipStream_t stream) {
  return launch(input, input_strides, input_neg, direction, direction_strides, direction_neg, out, dtype, batch, n,
                variant, s_out, stream);
}

int fh_expm_params(const void* input, const int64_t input_strides[3], int input_neg, const void* direction,
                   const int64_t direction_strides[3], int direction_neg, int dtype, int64_t batch, int n,
                   int32_t* params, double* norms, hipStream_t stream) {
  int rc = validate(input, input_strides, dtype, batch, n, params);
  if (rc != FH_OK) return rc;
  const bool pair = direction != nullptr;
  if (pair && batch > 0 && direction_strides == nullptr) return fail(FH_ERR_INVALID_ARGUMENT, kDirectionMessage);
  if (batch == 0) return FH_OK;
  fh::ExpmArgs args;
  args.x = make_operand(input, input_strides, input_neg, dtype, n);
  args.g = pair ? make_operand(direction, direction_strides, direction_neg, dtype, n) : args.x;
  args.out = nullptr;
  args.s_out = nullptr;
  args.batch = batch;
  args.n = n;
  const hipError_t err = fh::launch_params(args, dtype, pair, params, norms, stream);
  if (err != hipSuccess) return fail(FH_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(err));
  g_error.clear();
  return FH_OK;
}

int fh_hc_mix(const void* h, const int64_t h_strides[3], int h_neg, const void* x, const int64_t x_strides[3],
              void* y, float* e_out, int dtype, int64_t batch, int n, int64_t cols, hipStream_t stream) {
  int rc = validate_hc(h, h_strides, x, x_strides, nullptr, nullptr, y, dtype, batch, n, cols);
  if (rc != FH_OK || batch == 0) return rc;
  const hipError_t err = fh::launch_hc_mix(fh::hc_operand(h, h_strides, h_neg, dtype), x, x_strides, nullptr,
                                           nullptr, y, nullptr, e_out, dtype, batch, n, cols, stream);
  if (err != hipSuccess) return fail(FH_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(err));
  g_error.clear();
  return FH_OK;
}

int fh_hc_mix_backward(const void* h, const int64_t h_strides[3], int h_neg, const void* x,
                       const int64_t x_strides[3], const void* grad, const int64_t grad_strides[3], void* dh,
                       void* dx, float* de_out, int dtype, int64_t batch, int n, int64_t cols, hipStream_t stream) {
  int rc = validate_hc(h, h_strides, x, x_strides, grad, grad_strides, dx, dtype, batch, n, cols);
  if (rc != FH_OK) return rc;
  if (batch > 0 && (grad == nullptr || dh == nullptr))
    return fail(FH_ERR_INVALID_ARGUMENT, "hc_mix: null grad or dh pointer");
  if (batch == 0) return FH_OK;
  const hipError_t err = fh::launch_hc_mix(fh::hc_operand(h, h_strides, h_neg, dtype), x, x_strides, grad,
                                           grad_strides, dx, dh, de_out, dtype, batch, n, cols, stream);
  if (err != hipSuccess) return fail(FH_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(err));
  g_error.clear();
  return FH_OK;
}

int fh_hc_apply(const float* e, const void* x, const int64_t x_strides[3], void* y, int dtype, int64_t batch, int n,
                int64_t cols, hipStream_t stream) {
  g_error.clear();
  const int rc = validate_apply(e, x, x_strides, nullptr, nullptr, y, dtype, batch, n, cols);
  if (rc != FH_OK || batch == 0) return rc;
  const hipError_t err =
      fh::launch_hc_apply(e, x, x_strides, nullptr, nullptr, y, nullptr, dtype, batch, n, cols, stream);
  if (err != hipSuccess) return fail(FH_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FH_OK;
}

int fh_hc_apply_backward(const float* e, const void* x, const int64_t x_strides[3], const void* grad,
                         const int64_t grad_strides[3], void* dx, float* de, int dtype, int64_t batch, int n,
                         int64_t cols, hipStream_t stream) {
  g_error.clear();
  const int rc = validate_apply(e, x, x_strides, grad, grad_strides, dx, dtype, batch, n, cols);
  if (rc != FH_OK) return rc;
  if (batch > 0 && (grad == nullptr || de == nullptr))
    return fail(FH_ERR_INVALID_ARGUMENT, "hc_apply: null grad or de pointer");
  if (batch > 0 && !aligned(de, 4)) return fail(FH_ERR_INVALID_ARGUMENT, "hc_apply: dE must be 4-byte aligned float32");
  if (batch == 0) return FH_OK;
  const hipError_t err = fh::launch_hc_apply(e, x, x_strides, grad, grad_strides, dx, de, dtype, batch, n, cols, stream);
  if (err != hipSuccess) return fail(FH_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FH_OK;
}

const char* fh_last_error(void) { return g_error.c_str(); }

const char* fh_version(void) { return "0.1.0"; }

}  // extern "C"

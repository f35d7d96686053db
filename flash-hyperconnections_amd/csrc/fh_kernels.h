// Internal launcher declarations shared by the C-ABI entry points.
#pragma once

#include "fh_common.h"

namespace fh {

// Workgroups of `block` threads of `kernel` the current device holds at once
// (occupancy x compute units); at least 1.
int64_t resident_blocks(const void* kernel, int block);

// One wavefront per matrix, reference evaluation order (checking aid).
hipError_t launch_generic(const ExpmArgs& args, int dtype, int P, bool pair, hipStream_t stream);
// P == 4: one matrix per lane, 64 per wavefront, plain FP32 FMAs.
hipError_t launch_p4(const ExpmArgs& args, int dtype, bool pair, hipStream_t stream);
// P == 8: 4x4x1 MFMA blocks; the forward with 16 matrices per wavefront
// (launch_oct16), the Frechet derivative with 4.
hipError_t launch_oct(const ExpmArgs& args, int dtype, bool pair, hipStream_t stream);
hipError_t launch_oct16(const ExpmArgs& args, int dtype, hipStream_t stream);
// P in {16, 32}: one wavefront per matrix on 16x16x4 / 32x32x2 MFMA.
hipError_t launch_tile(const ExpmArgs& args, int dtype, int P, bool pair, hipStream_t stream);
// Fused hyper-connection stream mixing (n = 2..4): gy == nullptr selects the
// forward Y = exp(H) X into `out`; otherwise the backward dX = exp(H)^T dY into
// `out` and dH = L(H^T, dY X^T) into `dh`.  `xs` / `gs`: element strides
// (token, row) of X / dY, whose columns are contiguous.  `aux` (may be null):
// FP32 [B, n, n] copy of exp(H) (forward) or dY X^T (backward).
// H of the stream mixing as an element-class operand.
Operand hc_operand(const void* h, const int64_t strides[3], int neg, int dtype);
hipError_t launch_hc_mix(const Operand& h, const void* x, const int64_t* xs, const void* gy, const int64_t* gs,
                         void* out, void* dh, float* aux, int dtype, int64_t batch, int n, int64_t cols,
                         hipStream_t stream);
// exp(H) supplied in FP32 (5 <= n <= 8): gy == nullptr applies it (out = E X);
// otherwise out = E^T dY and de = dY X^T (FP32).
hipError_t launch_hc_apply(const float* e, const void* x, const int64_t* xs, const void* gy, const int64_t* gs,
                           void* out, float* de, int dtype, int64_t batch, int n, int64_t cols, hipStream_t stream);
// (degree, s) and FP64 norm per matrix.
hipError_t launch_params(const ExpmArgs& args, int dtype, bool pair, int32_t* params, double* norms,
                         hipStream_t stream);

}  // namespace fh

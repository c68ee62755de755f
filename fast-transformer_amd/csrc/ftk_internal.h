// Internal launch interface between the C-ABI layer (ftk_capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ftk_plan.h"

namespace ftk {

// Arguments of one skinny projection launch (GEMV or MFMA kind).
struct ProjArgs {
  const uint16_t* x;      // [M, K] BF16, row-major, 16-byte aligned
  const uint16_t* w;      // [N, K] BF16 (PyTorch Linear layout), 16-byte aligned
  const uint16_t* gamma;  // [K] RMSNorm gain, or null (no prologue)
  uint16_t* y;            // STORE: [M, N]; SWIGLU: [M, N/2]; ARGMAX: logits [M, N] or null
  float eps;
  int M, N, K;
  // EPI_ARGMAX only
  void* ids;              // [M] int32 or int64
  int ids_bytes;
  float* top;             // [M] winning logit as FP32, or null
  unsigned long long* keys;  // [M] zeroed workspace (left zeroed on exit)
  unsigned int* ticket;      // zeroed workspace counter (left zeroed on exit)
};

// Launch shape of the GEMV kind.
struct GemvShape {
  int rpw;       // weight rows per wave per tile (even for SwiGLU)
  int unroll;    // 16-byte chunks per lane issued per batch of loads
  int grid;      // workgroups (grid-stride over tiles)
  int tiles;
  size_t lds;    // dynamic LDS bytes (x staged as BF16)
};

// Device properties the planner needs (cached per device).
struct DeviceInfo {
  int cus;
  int lds_per_group_max;
  int ok;
};
DeviceInfo device_info();

bool gemv_supported(int M, int rpw, int unroll, int epi);
hipError_t launch_gemv(const ProjArgs& a, int epi, const GemvShape& shape, hipStream_t stream);

// Ragged or unaligned shapes: one wave per weight row, scalar loads, no prologue/epilogue.
hipError_t launch_gemm_generic(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N, int K,
                               hipStream_t stream);

// Standalone operators (the reference's separate kernels).
hipError_t launch_rms_norm(const uint16_t* x, int64_t row_stride, const uint16_t* gamma, uint16_t* y, int rows,
                           int cols, float eps, hipStream_t stream);
hipError_t launch_add_rms_norm(const void* x, int splits, int64_t split_stride, const uint16_t* residual,
                               const uint16_t* gamma, uint16_t* y, uint16_t* sum, int rows, int cols, float eps,
                               hipStream_t stream);
hipError_t launch_swiglu(const void* packed, int splits, int64_t split_stride, uint16_t* out, int rows, int width,
                         hipStream_t stream);
hipError_t launch_argmax(const uint16_t* logits, int rows, int vocab, void* ids, int ids_bytes, float* top,
                         unsigned long long* keys, unsigned int* ticket, hipStream_t stream);
hipError_t launch_merge_splits(const float* partial, int splits, int64_t count, uint16_t* out, hipStream_t stream);

}  // namespace ftk

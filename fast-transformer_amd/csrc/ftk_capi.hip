// extern "C" entry points of libftk.so (declared in include/ftk.h): argument
// checks, launch planning and dispatch to the gfx950 kernels.
#include <stdint.h>
#include <string.h>

#include "../../include/ftk.h"
#include "ftk_internal.h"

namespace ftk {

static thread_local int g_last_hip_error = 0;

static int hip_status(hipError_t e) {
  if (e == hipSuccess) return FTK_OK;
  g_last_hip_error = (int)e;
  return FTK_ERR_HIP;
}

DeviceInfo device_info() {
  static DeviceInfo cache[64];
  int dev = 0;
  DeviceInfo none = {0, 0, 0};
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return none;
  DeviceInfo& d = cache[dev];
  if (!d.ok) {
    int cus = 0, lds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return none;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) lds = 65536;
    d.cus = cus;
    d.lds_per_group_max = lds;
    d.ok = 1;
  }
  return d;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Planner defaults for the GEMV kind.
constexpr int kDefaultRpw = 4;
constexpr int kDefaultUnroll = 2;
constexpr int kDefaultGroupsPerCu = 8;

static int plan(int64_t M, int64_t N, int64_t K, int epi, int cus, const ftk_config* cfg, ftk_plan* p) {
  memset(p, 0, sizeof(*p));
  if (M < 1 || M > FTK_MAX_ROWS || N < 1 || K < 1 || cus < 1) return FTK_ERR_INVALID;
  if (N > INT32_MAX / 2 || K > INT32_MAX / 2) return FTK_ERR_INVALID;
  if (epi < FTK_EPI_STORE || epi > FTK_EPI_ARGMAX) return FTK_ERR_INVALID;
  if (epi == FTK_EPI_SWIGLU && (N % 2)) return FTK_ERR_INVALID;
  int kind = cfg && cfg->kind ? cfg->kind : FTK_KIND_AUTO;
  if (kind == FTK_KIND_AUTO) kind = (K % 8 == 0 && M <= 4) ? FTK_KIND_GEMV : FTK_KIND_GENERIC;
  p->kind = kind;
  p->threads = kThreads;
  if (kind == FTK_KIND_GENERIC) {
    if (epi != FTK_EPI_STORE) return FTK_ERR_UNSUPPORTED;
    p->tiles = (int)((N + kWaves - 1) / kWaves);
    p->grid = p->tiles;
    p->rows_per_wave = 1;
    p->unroll = 1;
    return FTK_OK;
  }
  if (kind == FTK_KIND_GEMV) {
    if (K % 8 != 0 || M > 4) return FTK_ERR_UNSUPPORTED;
    const int rpw = cfg && cfg->rows_per_wave ? cfg->rows_per_wave : kDefaultRpw;
    const int unroll = cfg && cfg->unroll ? cfg->unroll : kDefaultUnroll;
    const int gpc = cfg && cfg->groups_per_cu ? cfg->groups_per_cu : kDefaultGroupsPerCu;
    if (!gemv_supported((int)M, rpw, unroll, epi)) return FTK_ERR_INVALID;
    if (epi == FTK_EPI_SWIGLU && rpw % 2) return FTK_ERR_INVALID;
    p->rows_per_wave = rpw;
    p->unroll = unroll;
    p->tiles = gemv_tiles(epi, (int)N, rpw);
    const int64_t cap = (int64_t)gpc * cus;
    p->grid = (int)(p->tiles < cap ? p->tiles : cap);
    p->lds_bytes = M * K * 2;
    if (p->lds_bytes > 160 * 1024) return FTK_ERR_UNSUPPORTED;
    return FTK_OK;
  }
  return FTK_ERR_UNSUPPORTED;
}

}  // namespace ftk

using namespace ftk;

extern "C" {

const char* ftk_version(void) { return "ftk 0.1 gfx950"; }

const char* ftk_status_string(int status) {
  switch (status) {
    case FTK_OK: return "ok";
    case FTK_ERR_INVALID: return "invalid argument";
    case FTK_ERR_UNSUPPORTED: return "shape or alignment not supported by this entry point";
    case FTK_ERR_WORKSPACE: return "workspace missing or too small";
    case FTK_ERR_HIP: return "HIP launch failed";
  }
  return "unknown status";
}

int ftk_last_hip_error(void) { return g_last_hip_error; }

int ftk_device_compute_units(void) {
  DeviceInfo d = device_info();
  return d.ok ? d.cus : -1;
}

int64_t ftk_argmax_workspace_bytes(int64_t rows) { return rows < 1 ? 0 : 8 * rows + 8; }

int ftk_plan_project(int64_t M, int64_t N, int64_t K, int epilogue, int compute_units, const ftk_config* cfg,
                     ftk_plan* p) {
  if (p == nullptr) return FTK_ERR_INVALID;
  return plan(M, N, K, epilogue, compute_units, cfg, p);
}

int ftk_plan_coverage(const ftk_plan* p, int64_t N, int epilogue, int32_t* counts, int64_t outputs,
                      int64_t* max_row) {
  if (p == nullptr || counts == nullptr || max_row == nullptr) return FTK_ERR_INVALID;
  if (outputs != gemv_outputs(epilogue, (int)N)) return FTK_ERR_INVALID;
  memset(counts, 0, sizeof(int32_t) * outputs);
  *max_row = -1;
  if (p->kind == FTK_KIND_GENERIC) {
    for (int b = 0; b < p->grid; ++b)
      for (int w = 0; w < kWaves; ++w) {
        const int64_t row = (int64_t)b * kWaves + w;
        if (row < N) {
          counts[row] += 1;
          if (row > *max_row) *max_row = row;
        }
      }
    return FTK_OK;
  }
  if (p->kind != FTK_KIND_GEMV) return FTK_ERR_UNSUPPORTED;
  const int pw = gemv_per_wave(epilogue, p->rows_per_wave);
  const int halves = epilogue == FTK_EPI_SWIGLU ? 2 : 1;
  for (int b = 0; b < p->grid; ++b)
    for (int tile = b; tile < p->tiles; tile += p->grid)
      for (int w = 0; w < kWaves; ++w)
        for (int s = 0; s < pw; ++s) {
          const int col = gemv_output(tile, w, s, pw);
          const int clamped = col < outputs ? col : (int)outputs - 1;
          for (int h = 0; h < halves; ++h) {
            const int64_t row = gemv_weight_row(epilogue, clamped, h, (int)N);
            if (row > *max_row) *max_row = row;
          }
          if (col < outputs) counts[col] += 1;
        }
  return FTK_OK;
}

int ftk_project_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M, int64_t N,
                     int64_t K, int epilogue, void* ids, int ids_bytes, float* top, void* workspace,
                     int64_t workspace_bytes, const ftk_config* cfg, void* stream) {
  if (x == nullptr || w == nullptr) return FTK_ERR_INVALID;
  if (epilogue != FTK_EPI_ARGMAX && y == nullptr) return FTK_ERR_INVALID;
  if (epilogue == FTK_EPI_ARGMAX) {
    if (ids == nullptr || (ids_bytes != 4 && ids_bytes != 8)) return FTK_ERR_INVALID;
    if (workspace == nullptr || workspace_bytes < ftk_argmax_workspace_bytes(M)) return FTK_ERR_WORKSPACE;
  }
  DeviceInfo d = device_info();
  if (!d.ok) return hip_status(hipErrorNoDevice);
  ftk_plan p;
  int st = plan(M, N, K, epilogue, d.cus, cfg, &p);
  if (st != FTK_OK) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (p.kind == FTK_KIND_GENERIC) {
    if (gamma != nullptr) return FTK_ERR_UNSUPPORTED;
    return hip_status(launch_gemm_generic((const uint16_t*)x, (const uint16_t*)w, (uint16_t*)y, (int)M, (int)N,
                                          (int)K, s));
  }
  if (!aligned16(x) || !aligned16(w) || (gamma && !aligned16(gamma))) return FTK_ERR_UNSUPPORTED;
  ProjArgs a;
  memset(&a, 0, sizeof(a));
  a.x = (const uint16_t*)x;
  a.w = (const uint16_t*)w;
  a.gamma = (const uint16_t*)gamma;
  a.y = (uint16_t*)y;
  a.eps = eps;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.ids = ids;
  a.ids_bytes = ids_bytes;
  a.top = top;
  if (epilogue == FTK_EPI_ARGMAX) {
    a.keys = (unsigned long long*)workspace;
    a.ticket = (unsigned int*)((char*)workspace + 8 * M);
  }
  GemvShape g = {p.rows_per_wave, p.unroll, p.grid, p.tiles, (size_t)p.lds_bytes};
  return hip_status(launch_gemv(a, epilogue, g, s));
}

int ftk_linear_bf16(const void* x, const void* w, void* y, int64_t M, int64_t N, int64_t K, void* stream) {
  if (x && w && (!aligned16(x) || !aligned16(w))) {
    ftk_config c = {FTK_KIND_GENERIC, 0, 0, 0};
    return ftk_project_bf16(x, nullptr, 0.f, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0, &c,
                            stream);
  }
  return ftk_project_bf16(x, nullptr, 0.f, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0, nullptr,
                          stream);
}

int ftk_rms_norm_linear_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M,
                             int64_t N, int64_t K, void* stream) {
  if (gamma == nullptr) return FTK_ERR_INVALID;
  if (K % 8 || M > 4) return FTK_ERR_UNSUPPORTED;
  return ftk_project_bf16(x, gamma, eps, w, y, M, N, K, FTK_EPI_STORE, nullptr, 0, nullptr, nullptr, 0, nullptr,
                          stream);
}

int ftk_gate_up_swiglu_bf16(const void* x, const void* gamma, float eps, const void* w, void* y, int64_t M,
                            int64_t I, int64_t K, void* stream) {
  if (K % 8 || M > 4) return FTK_ERR_UNSUPPORTED;
  return ftk_project_bf16(x, gamma, eps, w, y, M, 2 * I, K, FTK_EPI_SWIGLU, nullptr, 0, nullptr, nullptr, 0,
                          nullptr, stream);
}

int ftk_lm_head_argmax_bf16(const void* x, const void* gamma, float eps, const void* w, void* logits, void* ids,
                            int ids_bytes, float* top, int64_t M, int64_t V, int64_t K, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  if (K % 8 || M > 4) return FTK_ERR_UNSUPPORTED;
  return ftk_project_bf16(x, gamma, eps, w, logits, M, V, K, FTK_EPI_ARGMAX, ids, ids_bytes, top, workspace,
                          workspace_bytes, nullptr, stream);
}

int ftk_rms_norm_bf16(const void* x, int64_t row_stride, const void* gamma, void* y, int64_t rows, int64_t cols,
                      float eps, void* stream) {
  if (!x || !gamma || !y || rows < 1 || cols < 1 || row_stride < cols || rows > INT32_MAX || cols > INT32_MAX)
    return FTK_ERR_INVALID;
  return hip_status(launch_rms_norm((const uint16_t*)x, row_stride, (const uint16_t*)gamma, (uint16_t*)y, (int)rows,
                                    (int)cols, eps, reinterpret_cast<hipStream_t>(stream)));
}

int ftk_add_rms_norm_bf16(const void* x, int x_splits, int64_t x_split_stride, const void* residual,
                          const void* gamma, void* y, void* sum, int64_t rows, int64_t cols, float eps, void* stream) {
  if (!x || !residual || !gamma || !y || !sum || rows < 1 || cols < 1 || x_splits < 0 || rows > INT32_MAX ||
      cols > INT32_MAX)
    return FTK_ERR_INVALID;
  if (x_splits > 0 && x_split_stride < rows * cols) return FTK_ERR_INVALID;
  return hip_status(launch_add_rms_norm(x, x_splits, x_split_stride, (const uint16_t*)residual,
                                        (const uint16_t*)gamma, (uint16_t*)y, (uint16_t*)sum, (int)rows, (int)cols,
                                        eps, reinterpret_cast<hipStream_t>(stream)));
}

int ftk_swiglu_bf16(const void* packed, int splits, int64_t split_stride, void* out, int64_t rows, int64_t width,
                    void* stream) {
  if (!packed || !out || rows < 1 || width < 1 || splits < 0 || rows > INT32_MAX || width > INT32_MAX)
    return FTK_ERR_INVALID;
  if (splits > 0 && split_stride < 2 * rows * width) return FTK_ERR_INVALID;
  if (rows * width > (int64_t)UINT32_MAX * kThreads) return FTK_ERR_INVALID;
  return hip_status(launch_swiglu(packed, splits, split_stride, (uint16_t*)out, (int)rows, (int)width,
                                  reinterpret_cast<hipStream_t>(stream)));
}

int ftk_argmax_bf16(const void* logits, int64_t rows, int64_t vocab, void* ids, int ids_bytes, float* top,
                    void* workspace, int64_t workspace_bytes, void* stream) {
  if (!logits || !ids || rows < 1 || vocab < 1 || (ids_bytes != 4 && ids_bytes != 8)) return FTK_ERR_INVALID;
  if (rows > 65535 || vocab > INT32_MAX) return FTK_ERR_INVALID;
  if (workspace == nullptr || workspace_bytes < ftk_argmax_workspace_bytes(rows)) return FTK_ERR_WORKSPACE;
  unsigned long long* keys = (unsigned long long*)workspace;
  unsigned int* ticket = (unsigned int*)((char*)workspace + 8 * rows);
  return hip_status(launch_argmax((const uint16_t*)logits, (int)rows, (int)vocab, ids, ids_bytes, top, keys, ticket,
                                  reinterpret_cast<hipStream_t>(stream)));
}

int ftk_merge_splits_bf16(const float* partial, int64_t splits, int64_t count, void* out, void* stream) {
  if (!partial || !out || splits < 1 || count < 1 || splits > INT32_MAX) return FTK_ERR_INVALID;
  if (count > (int64_t)UINT32_MAX * kThreads) return FTK_ERR_INVALID;
  return hip_status(launch_merge_splits(partial, (int)splits, count, (uint16_t*)out,
                                        reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"

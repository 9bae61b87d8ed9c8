// C-ABI entry points for the quantized matmul and the library's error state.
#include <stdarg.h>
#include <stdio.h>

#include <map>
#include <mutex>
#include <utility>

#include "bmx_device.h"

namespace bmx {

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return BMX_OK;
  return set_error(static_cast<int>(e), "%s: %s", what, hipGetErrorString(e));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

int allow_lds_ptr(const void* kernel, size_t bytes) {
  // (device, kernel) -> dynamic LDS limit already set
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, size_t> raised;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(BMX_E_ARG, "no current HIP device");
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = raised[{dev, kernel}];
  if (bytes <= have) return BMX_OK;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)) != hipSuccess)
    return set_error(BMX_E_UNSUPPORTED, "kernel needs %zu bytes of LDS", bytes);
  have = bytes;
  return BMX_OK;
}

int resident_blocks(const void* kernel, int threads, size_t lds) {
  // (device, kernel, lds) -> workgroups resident on the whole device
  static std::mutex mu;
  static std::map<std::pair<std::pair<int, const void*>, size_t>, int> known;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  int& n = known[{{dev, kernel}, lds}];
  if (n > 0) return n;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess || per_cu < 1)
    per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
  n = per_cu * cus;
  return n;
}

}  // namespace bmx

using namespace bmx;

extern "C" const char* bmx_last_error(void) { return g_last_error; }

extern "C" int bmx_abi_version(void) { return (2 << 16) | 1; }

namespace {

// quantized_matmul for every entry point: ws (fp32 split-K partials) is the
// caller's workspace, or null for the library's per-stream buffer.
int qmatmul(const bmx_bf16* x, const uint32_t* w, const bmx_bf16* scales, const bmx_bf16* biases, bmx_bf16* y,
            int64_t M, int64_t N, int64_t K, int transpose, int group_size, int bits, float* ws, size_t ws_floats,
            hipStream_t stream) {
  if (!transpose)
    return set_error(BMX_E_UNSUPPORTED, "qmatmul: transpose=false is not supported (W must be [N, K/8], "
                                        "as every quantized_matmul call of the reference passes it)");
  if (bits != 4 || group_size != 64)
    return set_error(BMX_E_UNSUPPORTED, "qmatmul: only bits=4, group_size=64 (got %d, %d)", bits, group_size);
  if (!x || !w || !scales || !biases || !y) return set_error(BMX_E_ARG, "qmatmul: null pointer");
  if (M < 0 || N <= 0 || K <= 0 || K % 64 || N > INT32_MAX || K > INT32_MAX || M > INT32_MAX)
    return set_error(BMX_E_SHAPE, "qmatmul: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                     (long long)K);
  if (M == 0) return BMX_OK;
  if (M > 8)
    return launch_qmm(x, w, scales, biases, y, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), ws,
                      ws_floats, stream);
  QmvParams p{};
  p.ldx = K;
  p.nseg = 1;
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.seg[0] = QmvSegment{w, scales, biases, y, static_cast<int>(N), 0};
  p.x = x;
  p.m = static_cast<int>(M);
  p.part = ws;  // the K-split matrix-core GEMV's partials
  p.part_floats = ws_floats;
  return launch_qmv(p, QMV_STORE, stream);
}

}  // namespace

extern "C" int bmx_qmatmul_affine(const bmx_bf16* x, const uint32_t* w, const bmx_bf16* scales,
                                  const bmx_bf16* biases, bmx_bf16* y, int64_t M, int64_t N, int64_t K, int transpose,
                                  int group_size, int bits, void* stream) {
  return qmatmul(x, w, scales, biases, y, M, N, K, transpose, group_size, bits, nullptr, 0, as_stream(stream));
}

extern "C" size_t bmx_qmatmul_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 || N > INT32_MAX || K > INT32_MAX || M > INT32_MAX) return 0;
  if (M > 8) return qmm_need_floats(QMM_STORE, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K)) * 4;
  // the GEMV splits K only on the matrix-core path (large N x K)
  return qmvx_workspace_floats(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K)) * 4;
}

extern "C" int bmx_qmatmul_affine_ws(const bmx_bf16* x, const uint32_t* w, const bmx_bf16* scales,
                                     const bmx_bf16* biases, bmx_bf16* y, int64_t M, int64_t N, int64_t K,
                                     int transpose, int group_size, int bits, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (!workspace && workspace_bytes) return set_error(BMX_E_ARG, "qmatmul_ws: null workspace of %zu bytes", workspace_bytes);
  if (!aligned(workspace, 16)) return set_error(BMX_E_ALIGN, "qmatmul_ws: workspace must be 16-byte aligned");
  NoAllocScope no_alloc;
  return qmatmul(x, w, scales, biases, y, M, N, K, transpose, group_size, bits, static_cast<float*>(workspace),
                 workspace_bytes / sizeof(float), as_stream(stream));
}

// ---------------------------------------------------------------------------
// bmx_qmatmul_affine_noalloc: the split-K partials live in `scratch`, a
// file-scope device array of kScratchBytes that every device the library
// runs on holds from module load until the process ends.  Host code never
// uses the array's name as an address: its per-device address comes from
// hipGetSymbolAddress, taken once per device (with that device current) at
// the entry point's first call there.  Every split-K launch writes each
// partial it later reads, so nothing in the array needs clearing between
// calls; calls that overlap on one device share the array and race.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kScratchBytes = size_t{16} << 20;  // 16 MiB
constexpr int kMaxDevices = 64;

__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

int device_scratch(float** out) {
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "noalloc: hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return set_error(BMX_E_ARG, "noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "noalloc: hipGetSymbolAddress")) return rc;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return BMX_OK;
}

}  // namespace

extern "C" int bmx_qmatmul_affine_noalloc(const bmx_bf16* x, const uint32_t* w, const bmx_bf16* scales,
                                          const bmx_bf16* biases, bmx_bf16* y, int64_t M, int64_t N, int64_t K,
                                          int transpose, int group_size, int bits, void* stream) {
  const size_t need = bmx_qmatmul_workspace_bytes(M, N, K);
  if (need > kScratchBytes)
    return set_error(BMX_E_SHAPE, "qmatmul_noalloc: M=%lld N=%lld K=%lld needs %zu bytes of split-K scratch, "
                     "above the %zu-byte maximum",
                     (long long)M, (long long)N, (long long)K, need, kScratchBytes);
  float* ptr = nullptr;
  if (need > 0) {
    if (int rc = device_scratch(&ptr)) return rc;
  }
  NoAllocScope no_alloc;
  return qmatmul(x, w, scales, biases, y, M, N, K, transpose, group_size, bits, ptr,
                 ptr ? kScratchBytes / sizeof(float) : 0, as_stream(stream));
}

// Allocation-free form of qutai_amd_gemm for callers that cannot allocate
// device memory (code under HIP graph capture, serving loops, harnesses that
// forbid hipMalloc): the workspace that qutai_amd_gemm takes from its caller
// (operand re-layout, split-K partial sums) is a fixed array in device
// memory instead, one per GPU, held until the process ends.
#include <mutex>

#include <hip/hip_runtime.h>

#include "qutai_amd.h"

namespace {

constexpr size_t SCRATCH_BYTES = (size_t)128 << 20;
constexpr int MAX_DEVICES = 64;

// The name is a host-side handle only: host code uses the device address
// that hipGetSymbolAddress returns for the current GPU (scratch_address).
__device__ __align__(256) char scratch[SCRATCH_BYTES];

std::mutex scratch_lock;
void* scratch_ptr[MAX_DEVICES] = {};

// Device address of `scratch` on the current GPU, looked up once per device.
int scratch_address(void** ptr) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return (int)status;
  if (device < 0 || device >= MAX_DEVICES) return QA_EINVAL;
  std::lock_guard<std::mutex> guard(scratch_lock);
  if (!scratch_ptr[device]) {
    void* address = nullptr;
    status = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (status != hipSuccess) return (int)status;
    if (!address) return QA_EINVAL;
    scratch_ptr[device] = address;
  }
  *ptr = scratch_ptr[device];
  return QA_OK;
}

}  // namespace

extern "C" {

size_t qutai_amd_gemm_static_capacity(void) { return SCRATCH_BYTES; }

int qutai_amd_gemm_static(const void* a, const void* b, void* out, int64_t rows, int64_t inner, int64_t cols,
                          int64_t batch, int64_t left_stride, int64_t right_stride, int transpose_left,
                          int transpose_right, int a_dtype, int b_dtype, int out_dtype, int accumulate,
                          int bf16_compute, void* stream) {
  if (rows < 0 || inner < 0 || cols < 0 || batch < 0 || left_stride < 0 || right_stride < 0) return QA_EINVAL;
  // workspace need for these operands; unaligned bases add at most the
  // re-layout of an operand that the 256-byte-aligned estimate keeps in place
  size_t need = qutai_amd_gemm_workspace_size(rows, inner, cols, batch, left_stride, right_stride, transpose_left,
                                              transpose_right, a_dtype, b_dtype, bf16_compute);
  const bool misaligned = ((uintptr_t)a % 16) || ((uintptr_t)b % 16);
  if (need == 0 && !misaligned)  // operands used in place: no scratch at all
    return qutai_amd_gemm(a, b, out, rows, inner, cols, batch, left_stride, right_stride, transpose_left,
                          transpose_right, a_dtype, b_dtype, out_dtype, accumulate, bf16_compute, nullptr, 0,
                          stream);
  if (need > SCRATCH_BYTES) return QA_ESCRATCH;
  void* ptr = nullptr;
  const int status = scratch_address(&ptr);
  if (status != QA_OK) return status;
  // qutai_amd_gemm checks the exact need (incl. a misaligned base) against
  // the capacity and returns QA_EWORKSPACE when it does not fit
  const int result = qutai_amd_gemm(a, b, out, rows, inner, cols, batch, left_stride, right_stride, transpose_left,
                                    transpose_right, a_dtype, b_dtype, out_dtype, accumulate, bf16_compute, ptr,
                                    SCRATCH_BYTES, stream);
  return result == QA_EWORKSPACE ? QA_ESCRATCH : result;
}

}  // extern "C"

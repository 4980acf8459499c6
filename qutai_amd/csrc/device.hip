// Device identification for the host runtime: the architecture name comes
// from hipGetDeviceProperties through the HIP headers, so the host never has
// to know the layout of hipDeviceProp_t.
#include <string.h>

#include <hip/hip_runtime.h>

#include "qutai_amd.h"

extern "C" int qutai_amd_device_arch(int device, char* name, size_t size) {
  if (!name || size == 0) return QA_EINVAL;
  hipDeviceProp_t props;
  const hipError_t status = hipGetDeviceProperties(&props, device);
  if (status != hipSuccess) return (int)status;
  const size_t length = strnlen(props.gcnArchName, sizeof(props.gcnArchName));
  const size_t copied = length < size - 1 ? length : size - 1;
  memcpy(name, props.gcnArchName, copied);
  name[copied] = '\0';
  return QA_OK;
}

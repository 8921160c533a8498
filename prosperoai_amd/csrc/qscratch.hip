/*
 * The device scratch array of the no-allocation entry point
 * (pai_qgemm_f32_noalloc_async): a file-scope device array, so a call that
 * may not allocate still has room for the 16-bit copy of its activations.
 *
 * Each GPU that loads this library holds its own copy of the array, at its
 * own address, until the process ends. In host code the name `scratch` is
 * a host-side stand-in, not a device address: host code uses only the
 * address paik_scratch_address returns for the current device.
 */
#include <hip/hip_runtime.h>

#include "paik.h"

static __device__ __align__(256) uint8_t scratch[PAIK_SCRATCH_BYTES];

/* Device address of the current device's copy of the array (hipError_t as
 * int). Called once per device, with that device current. */
extern "C" int paik_scratch_address(void **ptr) {
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return (int)e;
  *ptr = p;
  return 0;
}

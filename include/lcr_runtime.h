/*
 * lcr_runtime.h — device memory and synchronisation helpers of the C-ABI.
 *
 * Not a counterpart of any reference interface: the reference's host code and
 * kernel tests call the CUDA runtime directly (cudaMalloc / cudaMemcpy /
 * cudaDeviceSynchronize, tests/test_kernels.cu:37-65). Hosts that drive this
 * library through its C-ABI alone (Python ctypes, cgo, JNI) get the same few
 * operations here, on the same HIP runtime instance the kernels use, so no
 * second GPU runtime has to be loaded into the process. Return values follow
 * lcr_kernels.h.
 */
#ifndef LCR_RUNTIME_H_
#define LCR_RUNTIME_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int lcr_device_malloc(void** out, size_t bytes);
int lcr_device_free(void* ptr);
int lcr_memcpy_htod(void* dst, const void* src, size_t bytes);
int lcr_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int lcr_memcpy_dtod(void* dst, const void* src, size_t bytes);
int lcr_device_memset(void* ptr, int value, size_t bytes);
int lcr_device_synchronize(void);

#ifdef __cplusplus
}
#endif

#endif /* LCR_RUNTIME_H_ */

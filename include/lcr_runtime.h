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

/* extension (measurement): reads `bytes` of device memory at `buf` (16-byte aligned, a multiple of
 * 16 KiB) with the streaming 16-byte loads the decode kernels use, in `blocks` workgroups of 256
 * threads, reps + 1 times on the default stream; *best_ms is the fastest of the last `reps`
 * launches (hipEvents). bytes / *best_ms is the read rate the device sustains for this load form:
 * the measured ceiling beside the published HBM peak. */
int lcr_stream_read(const void* buf, size_t bytes, int blocks, int reps, float* best_ms);

#ifdef __cplusplus
}
#endif

#endif /* LCR_RUNTIME_H_ */

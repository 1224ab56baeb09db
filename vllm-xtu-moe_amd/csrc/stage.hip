// Expert staging: batched asynchronous copies of whole experts between a
// host store (pinned host memory) or another device array and a device ring
// slot / resident pool slot.  One call moves one weight plane of n experts;
// each expert is one contiguous hipMemcpyAsync on the caller's stream, so a
// tile of experts is a handful of large DMA transfers on the copy engine.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xtu_common.hpp"

extern "C" {

// dst[i * dst_stride, + bytes) <- src[experts[i] * src_stride, + bytes) for i < n.
// `experts` is a host array.  Replaces the per-expert shard DMA of the
// reference's ring (copy_hostbuf_to_device / _dma_hostbuf_range,
// xiaotu_moe/csrc/binding.cpp:1368-1437, vllm_xiaotu_moe/gpu_prefill.py:1897).
hipError_t xtu_copy_experts(int n, const int32_t* experts, const void* src, long src_stride,
                            void* dst, long dst_stride, long bytes, hipStream_t stream) {
  XTU_CHECK_ARG(n >= 0 && bytes >= 0 && src_stride >= bytes && dst_stride >= bytes);
  XTU_CHECK_ARG(n == 0 || bytes == 0 || (experts && src && dst));
  for (int i = 0; i < n; ++i) {
    XTU_CHECK_ARG(experts[i] >= 0);
    if (bytes == 0) continue;
    const hipError_t e = hipMemcpyAsync(static_cast<uint8_t*>(dst) + (long)i * dst_stride,
                                        static_cast<const uint8_t*>(src) +
                                            (long)experts[i] * src_stride,
                                        (size_t)bytes, hipMemcpyDefault, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Pitched copy of `height` rows of `width` bytes (hipMemcpy2DAsync, any
// direction).  Replaces the engine's copy_hostbuf_to_device_2d
// (xiaotu_moe/csrc/python_binding/binding.cpp:1411-1435), which DMAs one NUMA
// node's shard rows straight into their strided place in a device slot.
hipError_t xtu_copy_2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                       size_t height, hipStream_t stream) {
  XTU_CHECK_ARG(width <= dpitch && width <= spitch);
  XTU_CHECK_ARG(width == 0 || height == 0 || (dst && src));
  if (width == 0 || height == 0) return hipSuccess;
  // the last row ends at (height - 1) * pitch + width on either side: reject
  // sizes whose span does not fit a size_t (a negative count cast to size_t)
  const size_t kMax = ~size_t(0);
  XTU_CHECK_ARG(height - 1 <= (kMax - width) / spitch && height - 1 <= (kMax - width) / dpitch);
  return hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDefault, stream);
}

}  // extern "C"

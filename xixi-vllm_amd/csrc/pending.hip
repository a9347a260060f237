// Entry points whose kernels are not built yet: they refuse every call.
#include <hip/hip_runtime.h>
#include "../../include/xv_kernels.h"
extern "C" int xv_prefill_attention(const void*, int64_t, int64_t, const void*, const void*, int64_t, int64_t,
                                    const void*, const void*, int64_t, int64_t, int64_t, const int32_t*, int64_t,
                                    const int32_t*, const int32_t*, void*, int64_t, int, int, int, int, int, int,
                                    float, hipStream_t) { return (int)hipErrorNotSupported; }
extern "C" size_t xv_sampler_workspace_size(int, int) { return 0; }
extern "C" int xv_sample(const void*, int64_t, int, int, const float*, const float*, const int32_t*, const float*,
                         const float*, int, int64_t*, void*, size_t, hipStream_t) { return (int)hipErrorNotSupported; }

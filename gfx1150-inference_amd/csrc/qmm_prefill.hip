// Prefill GEMM (M >= kGemvMaxM): dequantize weight tiles into LDS as bf16 and contract on MFMA.
#include "qmm_device.h"

namespace qmm {

bool gemm_prefill_supported(int, int, int, int, int, int, const void*, const void*, const void*) {
    return false;
}

hipError_t launch_gemm_prefill(int, const void*, int, const void*, void*, int, int, int, int, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace qmm

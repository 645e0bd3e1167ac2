// aih_qgemm.hip -- prefill GEMM with fused dequantization (MFMA).
#include "aih_internal.h"

int aih_launch_qgemm(aih_ctx *, int, const void *, int64_t, int64_t, const float *, int64_t, float *)
{
    return AIH_E_UNSUPPORTED;
}

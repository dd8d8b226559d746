// The activation staging kernel of the prefill matrix product (type-independent).
#include "gemv_impl.h"

namespace llmhip {

int prep_launch(const GemvArgs& a, int pro, hipStream_t s) {
  if ((uint64_t)a.nb * 4 > (uint64_t)PMAXI * 256)
    return set_error(LLMHIP_ERR_ARG, "llm: prep: k=%u is too long", a.k);
  dim3 grid(a.tg * 16);
  uint32_t lds = 0;
  switch (pro) {
    case PRO_PLAIN: hipLaunchKernelGGL(prep_kernel<PRO_PLAIN>, grid, dim3(256), lds, s, a); break;
    case PRO_RMS: hipLaunchKernelGGL(prep_kernel<PRO_RMS>, grid, dim3(256), lds, s, a); break;
    case PRO_PLAIN | PRO_Q8: hipLaunchKernelGGL(prep_kernel<PRO_PLAIN | PRO_Q8>, grid, dim3(256), lds, s, a); break;
    case PRO_RMS | PRO_Q8: hipLaunchKernelGGL(prep_kernel<PRO_RMS | PRO_Q8>, grid, dim3(256), lds, s, a); break;
    default: return set_error(LLMHIP_ERR_ARG, "llm: prep: prologue %d", pro);
  }
  LLM_HIP(hipGetLastError());
  return 0;
}

}  // namespace llmhip

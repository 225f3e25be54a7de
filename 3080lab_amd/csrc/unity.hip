// Single translation unit of libqwen355.so (the kernel templates are instantiated by the C ABI layer).
#include "gemv.hip"
#include "mmq.hip"
#include "mmq_q6k.hip"
#include "flash.hip"
#include "mega.hip"
#include "gemv_bf16.hip"
#include "gemm_f16.hip"
#include "capi.hip"

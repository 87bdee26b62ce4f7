// Instantiations of the f32-activation GEMV, BF16 weights.
#define VH_GEMV_WT vh::WT_BF16
#define VH_GEMV_INT false
#define VH_GEMV_ENTRY launch_gemv_flt_bf16
#include "vh_gemv_dispatch.hpp"

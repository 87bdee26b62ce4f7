// Instantiations of the f32-activation GEMV, F16 weights.
#define VH_GEMV_WT vh::WT_F16
#define VH_GEMV_INT false
#define VH_GEMV_ENTRY launch_gemv_flt_f16
#include "vh_gemv_dispatch.hpp"

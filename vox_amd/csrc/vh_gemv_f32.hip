// Instantiations of the f32-activation GEMV, F32 weights.
#define VH_GEMV_WT vh::WT_F32
#define VH_GEMV_INT false
#define VH_GEMV_ENTRY launch_gemv_flt_f32
#include "vh_gemv_dispatch.hpp"

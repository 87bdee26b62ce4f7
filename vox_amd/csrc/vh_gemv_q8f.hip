// Instantiations of the f32-activation GEMV, Q8 weights (m > 8).
#define VH_GEMV_WT vh::WT_Q8
#define VH_GEMV_INT false
#define VH_GEMV_ENTRY launch_gemv_flt_q8
#include "vh_gemv_dispatch.hpp"

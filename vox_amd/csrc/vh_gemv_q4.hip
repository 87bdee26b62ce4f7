// Instantiations of the int8-activation GEMV, Q4 weights.
#define VH_GEMV_WT vh::WT_Q4
#define VH_GEMV_INT true
#define VH_GEMV_ENTRY launch_gemv_int_q4
#include "vh_gemv_dispatch.hpp"

// Instantiations of the int8-activation GEMV, Q8 weights (decode, m <= 8).
#define VH_GEMV_WT vh::WT_Q8
#define VH_GEMV_INT true
#define VH_GEMV_ENTRY launch_gemv_int_q8
#include "vh_gemv_dispatch.hpp"

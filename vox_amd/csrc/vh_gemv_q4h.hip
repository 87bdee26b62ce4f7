// Instantiations of the int8-activation GEMV, Q4 weights with f16 block scales.
#define VH_GEMV_WT vh::WT_Q4H
#define VH_GEMV_INT true
#define VH_GEMV_ENTRY launch_gemv_int_q4h
#include "vh_gemv_dispatch.hpp"

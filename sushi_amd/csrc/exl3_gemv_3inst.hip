// GEMV kernels of one codebook family (the body is exl3_gemv_body.h; one family per translation unit so the
// template instantiations build in parallel).
#define EXL3_GEMV_FAM FAM_3INST
#include "exl3_gemv_body.h"

// kernels.hip — the single translation unit that becomes the gfx950 code
// object (runit_kernels.hsaco) loaded by the host runtime with hipModuleLoad.
#include "k_gemv.hip"
#include "k_gemv_ls.hip"
#include "k_aux.hip"
#include "k_decode.hip"
#include "k_gemm.hip"
#include "k_scratch.hip"
#include "k_step.hip"

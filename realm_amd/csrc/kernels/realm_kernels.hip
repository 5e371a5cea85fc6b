// Single translation unit for the gfx950 code object (realm_kernels.hsaco)
// that the host library embeds and loads with hipModuleLoadData.
#include "dequant.hip"
#include "gemv.hip"
#include "gemm.hip"
#include "dense.hip"

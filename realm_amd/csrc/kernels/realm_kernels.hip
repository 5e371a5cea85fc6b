// Translation unit of the non-GEMV kernels (dequant/repack, MFMA GEMM,
// dense, the element-wise layer operations).  The GEMV variants are compiled per weight format from
// gemv_fmt.hip, in parallel; the host library embeds every code object and
// loads each with hipModuleLoadData.
#include "dequant.hip"
#include "gemm.hip"
#include "dense.hip"
#include "layer_ops.hip"
#include "stream.hip"

// er_kernels.hip -- single translation unit of every gfx950 kernel, compiled
// with `hipcc --genco --offload-arch=gfx950` into one code object that the
// host library embeds and loads with hipModuleLoadData.
#include "er_dequant.hip"
#include "er_gemv.hip"
#include "er_gemm.hip"
#include "er_quant.hip"
#include "er_scratch.hip"
#include "er_probe.hip"

// er_kernels.hip -- single translation unit of every gfx950 kernel, compiled
// with `hipcc --genco --offload-arch=gfx950` into one code object that the
// host library embeds and loads with hipModuleLoadData.  Built a second time
// with -DER_WITH_PROBES for the measurement library (the product kernels
// plus probes and clock-stamped GEMM copies).
#include "er_dequant.hip"
#include "er_gemv.hip"
#include "er_gemm.hip"
#include "er_quant.hip"
#include "er_scratch.hip"
#ifdef ER_WITH_PROBES
// the measurement build only (libedgerunner_probe.so, bench.py's ceilings):
// streaming-read, launch, barrier, LDS and MFMA/VALU probes
#include "er_probe.hip"
#endif

// Single translation unit of the ds41 gfx950 library: every kernel shares the
// file-scope device status word without relocatable device code.
#include "moe_kernels.inc"
#include "moe_layer.inc"
#include "prefill.inc"
#include "dense_fp8.inc"
#include "target_experts.inc"
#include "expert_pool.inc"
#include "verify_stack.inc"
#include "expert_records.inc"
#include "accept.inc"
#include "spark_host.inc"
#include "spark_gpu.inc"
#include "read_probe.inc"

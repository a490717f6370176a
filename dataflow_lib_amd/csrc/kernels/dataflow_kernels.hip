/*
 * Single translation unit for the gfx950 code object loaded by the HIP
 * backend with hipModuleLoad (the reference builds one cubin the same way,
 * src/ops/nvidia/cuda_kernels.cu:4-20).
 */
#include "rms_norm.hip"
#include "rope.hip"
#include "swiglu.hip"
#include "softmax_xent.hip"
#include "gather_scatter.hip"
#include "fp8_ops.hip"

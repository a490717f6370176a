/*
 * ABI of the launch-configuration library (dlopen'ed by the HIP backend).
 * One "<op>_set_launch_config" per op family, plus the attribute inits of the
 * RMSNorm and softmax families (reference: src/ops/nvidia/include/nvidia_ops_config.h:9-27).
 * Each returns 0, or -1 when the op cannot be launched for these arguments.
 */
#ifndef HIP_OPS_CONFIG_H
#define HIP_OPS_CONFIG_H

#include "dataflow_common.h"
#include "ops.h"
#include "dataflow_handle.h"
#include "hip_dataflow_handle.h"

#ifdef __cplusplus
extern "C" {
#endif

int rms_norm_set_attribute_config(Dataflow_Handle * dataflow_handle, Hip_Function * hip_function);
int rms_norm_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);

int rms_norm_bwd_x_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
int rms_norm_bwd_w_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
int rms_norm_bwd_w_set_finish_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
/* fused exact-gradient backward (no reference counterpart) */
int rms_norm_bwd_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
int rms_norm_bwd_set_finish_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);

/* src/ops/nvidia/preprocess/embedding_config.c:3-40 */
int embedding_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
/* src/ops/nvidia/attention/attn_misc_config.c:56-80 */
int copy_to_seq_context_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);

int rope_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
int rope_bwd_x_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
/* no reference counterpart: RoPE fused with the KV-cache scatter */
int rope_copy_to_seq_context_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);

int swiglu_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
int swiglu_bwd_x_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);

int softmax_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
int cross_entropy_loss_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
/* fused softmax + cross-entropy (no reference counterpart) */
int softmax_cross_entropy_loss_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);
/* attribute init of softmax and the fused op: flags the kernels that keep
 * launch-wide state in the code object (shares_module_scratch) */
int softmax_set_attribute_config(Dataflow_Handle * dataflow_handle, Hip_Function * hip_function);

#ifdef __cplusplus
}
#endif

#endif

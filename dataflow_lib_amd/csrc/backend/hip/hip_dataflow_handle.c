/*
 * HIP backend of Dataflow_Handle (COMPUTE_HSA) for gfx950.
 *
 * Behaviour follows the CUDA backend it replaces
 * (reference: src/dataflow_handle/nvidia/src/cuda_dataflow_handle.c:53-918,
 *  src/dataflow_handle/nvidia/src/cuda_drv.c), on HIP's runtime API:
 *  - native code: a gfx950 code object loaded with hipModuleLoad; every
 *    function record is keyed by the op's SHA-256 fingerprint;
 *  - launch geometry: "<op>_set_launch_config" from a dlopen'ed library;
 *  - submit_op: hipModuleLaunchKernel with kernelParams = op->op_args, then
 *    the optional "_finish" kernel of two-pass ops on the same stream;
 *  - streams: non-blocking, default priority; one timing-free event each.
 * Fixed relative to the reference: submit_peer_transfer is a device-to-device
 * copy from src to dest (cuda_dataflow_handle.c:912, cuda_drv.c:540,557), and
 * the device info reads the per-block thread limit (:689).
 */
#include "hip_dataflow_handle.h"
#include "fingerprint.h"

#define HIP_CHECK_RET(call, ret, ...) do { \
		hipError_t _e = (call); \
		if (_e != hipSuccess) { \
			fprintf(stderr, "hip backend: %s returned %s; ", #call, hipGetErrorString(_e)); \
			fprintf(stderr, __VA_ARGS__); \
			fprintf(stderr, "\n"); \
			return ret; \
		} \
	} while (0)

static uint64_t hip_op_table_hash_func(void * op_fingerprint, uint64_t table_size) {
	return fingerprint_to_least_sig64((uint8_t *) op_fingerprint, OP_IDENTIFIER_FINGERPRINT_NUM_BYTES) % table_size;
}

/* stream_id -1 is the NULL stream; anything else must name a created stream */
static int resolve_stream(Dataflow_Handle * h, int stream_id, hipStream_t * out, const char * what) {
	if (stream_id == -1) {
		*out = NULL;
		return 0;
	}
	if (stream_id < 0 || stream_id >= h->num_streams) {
		fprintf(stderr, "hip backend: stream id %d (for %s) is out of range: the handle has %d streams, and -1 names the null stream\n",
				stream_id, what, h->num_streams);
		return -1;
	}
	*out = ((hipStream_t *) h->streams)[stream_id];
	return 0;
}

/* ---------- 0. ops ---------- */

static int hip_register_native_code(Dataflow_Handle * dataflow_handle, char * native_code_filename, char * native_code_config_lib_filename,
									int num_funcs, Op_Skeleton * func_op_skeletons, char ** func_symbols, char ** func_set_launch_symbols, char ** func_init_symbols) {
	if (dataflow_handle->num_native_function_libs >= MAX_NATIVE_FUNCTION_LIBS) {
		fprintf(stderr, "hip backend: the handle already holds the maximum of %d native code objects\n", MAX_NATIVE_FUNCTION_LIBS);
		return -1;
	}
	HIP_CHECK_RET(hipSetDevice(dataflow_handle->device_id), -1, "device %d", dataflow_handle->device_id);

	hipModule_t * module = (hipModule_t *) malloc(sizeof(hipModule_t));
	if (!module) {
		fprintf(stderr, "hip backend: out of host memory for a module record\n");
		return -1;
	}
	hipError_t err = hipModuleLoad(module, native_code_filename);
	if (err != hipSuccess) {
		fprintf(stderr, "hip backend: hipModuleLoad could not load the code object %s (%s)\n", native_code_filename, hipGetErrorString(err));
		free(module);
		return -1;
	}

	void * config_lib = dlopen(native_code_config_lib_filename, RTLD_LAZY | RTLD_LOCAL);
	if (!config_lib) {
		fprintf(stderr, "hip backend: dlopen could not open the launch-config library %s (%s)\n",
				native_code_config_lib_filename, dlerror());
		hipModuleUnload(*module);
		free(module);
		return -1;
	}

	int added = 0;
	for (int i = 0; i < num_funcs; i++) {
		char * sym = func_symbols[i];
		if (!sym) {
			continue;
		}
		if (!func_set_launch_symbols[i]) {
			fprintf(stderr, "hip backend: native function %s has no launch-config symbol; skipped\n", sym);
			continue;
		}

		Hip_Function f;
		memset(&f, 0, sizeof(f));
		f.is_native = true;

		err = hipModuleGetFunction(&f.function_handle, *module, sym);
		if (err != hipSuccess) {
			fprintf(stderr, "hip backend: kernel #%d (%s) is not in the code object (%s); skipped\n", i, sym, hipGetErrorString(err));
			continue;
		}

		int max_threads = 0;
		if (hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f.function_handle) != hipSuccess || max_threads <= 0) {
			max_threads = ((Hip_Device_Info *) dataflow_handle->device_info)->max_threads_per_block;
		}
		f.function_config.func_max_threads_per_block = MY_MIN(max_threads, HIP_DEV_UPPER_BOUND_MAX_THREADS_ALL_FUNC);
		f.function_config.func_max_smem = ((Hip_Device_Info *) dataflow_handle->device_info)->max_smem_per_block;

		f.set_launch_config = (Hip_Set_Launch_Config) dlsym(config_lib, func_set_launch_symbols[i]);
		if (!f.set_launch_config) {
			fprintf(stderr, "hip backend: kernel #%d (%s): launch-config symbol %s is not in the launch-config library; skipped\n",
					i, sym, func_set_launch_symbols[i]);
			continue;
		}

		/* optional second pass: "<sym>_finish" + "<op>_set_finish_launch_config" */
		char finish_sym[FUNC_SYMBOL_MAX_LEN + 16];
		snprintf(finish_sym, sizeof(finish_sym), "%s_finish", sym);
		hipFunction_t finish_fn = NULL;
		if (hipModuleGetFunction(&finish_fn, *module, finish_sym) == hipSuccess && finish_fn) {
			const char * suffix = "_set_launch_config";
			size_t len = strlen(func_set_launch_symbols[i]);
			size_t slen = strlen(suffix);
			char finish_cfg[FUNC_SYMBOL_MAX_LEN + 32];
			if (len <= slen || strcmp(func_set_launch_symbols[i] + len - slen, suffix) != 0) {
				fprintf(stderr, "hip backend: launch-config symbol %s of two-kernel function %s does not end in %s; skipped\n", func_set_launch_symbols[i], sym, suffix);
				continue;
			}
			snprintf(finish_cfg, sizeof(finish_cfg), "%.*s_set_finish_launch_config", (int) (len - slen), func_set_launch_symbols[i]);
			f.set_finish_launch_config = (Hip_Set_Launch_Config) dlsym(config_lib, finish_cfg);
			if (!f.set_finish_launch_config) {
				fprintf(stderr, "hip backend: %s has a second kernel but the launch-config library lacks %s; skipped\n", sym, finish_cfg);
				continue;
			}
			f.finish_function_handle = finish_fn;
		}
		else {
			/* clear the sticky "not found" status of the failed lookup */
			(void) hipGetLastError();
		}

		memcpy(&f.op_skeleton, &func_op_skeletons[i], sizeof(Op_Skeleton));
		f.hip_external_func = NULL;
		f.op_extra = NULL;

		/* the init sees the whole record (skeleton and second kernel included) */
		if (func_init_symbols && func_init_symbols[i]) {
			Hip_Set_Func_Attribute init_fn = (Hip_Set_Func_Attribute) dlsym(config_lib, func_init_symbols[i]);
			if (!init_fn) {
				fprintf(stderr, "hip backend: kernel #%d (%s): init symbol %s is not in the launch-config library; skipped\n",
						i, sym, func_init_symbols[i]);
				continue;
			}
			if (init_fn(dataflow_handle, &f)) {
				fprintf(stderr, "hip backend: kernel #%d (%s): init %s reported an error; skipped\n",
						i, sym, func_init_symbols[i]);
				continue;
			}
		}

		if (insert_table(&dataflow_handle->op_table, f.op_skeleton.identifier.fingerprint, &f)) {
			fprintf(stderr, "hip backend: kernel #%d (%s) could not be added to the op table; skipped\n", i, sym);
			continue;
		}
		added++;
	}

	if (added == 0) {
		fprintf(stderr, "hip backend: none of the requested functions could be registered\n");
		dlclose(config_lib);
		hipModuleUnload(*module);
		free(module);
		return -1;
	}

	dataflow_handle->native_function_libs[dataflow_handle->num_native_function_libs++] = module;
	dataflow_handle->num_ops += added;
	return added;
}

static int hip_register_external_code(Dataflow_Handle * dataflow_handle, char * external_code_filename, int num_funcs,
									Op_Skeleton * func_op_skeletons, char ** func_symbols, char ** func_init_symbols) {
	void * lib = dlopen(external_code_filename, RTLD_LAZY | RTLD_LOCAL);
	if (!lib) {
		fprintf(stderr, "hip backend: dlopen could not open the external op library %s (%s)\n", external_code_filename, dlerror());
		return -1;
	}
	int added = 0;
	for (int i = 0; i < num_funcs; i++) {
		char * sym = func_symbols[i];
		if (!sym) {
			continue;
		}
		Hip_Function f;
		memset(&f, 0, sizeof(f));
		f.hip_external_func = (int (*)(Dataflow_Handle *, int, Op *, void *)) dlsym(lib, sym);
		if (!f.hip_external_func) {
			fprintf(stderr, "hip backend: symbol %s is not in the external op library %s; skipped\n", sym, external_code_filename);
			continue;
		}
		if (func_init_symbols && func_init_symbols[i]) {
			External_Lib_Func_Init init_fn = (External_Lib_Func_Init) dlsym(lib, func_init_symbols[i]);
			if (!init_fn) {
				fprintf(stderr, "hip backend: init symbol %s of external function %s not found; skipped\n", func_init_symbols[i], sym);
				continue;
			}
			if (init_fn(dataflow_handle, (void *) &f)) {
				fprintf(stderr, "hip backend: init %s of external function %s reported an error; skipped\n", func_init_symbols[i], sym);
				continue;
			}
		}
		memcpy(&f.op_skeleton, &func_op_skeletons[i], sizeof(Op_Skeleton));
		f.is_native = false;
		if (insert_table(&dataflow_handle->op_table, f.op_skeleton.identifier.fingerprint, &f)) {
			fprintf(stderr, "hip backend: kernel #%d (%s) could not be added to the op table; skipped\n", i, sym);
			continue;
		}
		added++;
	}
	dataflow_handle->num_ops += added;
	return added;
}

/* ---------- 1. compute ---------- */

static int launch(hipFunction_t fn, Hip_Launch_Config * cfg, hipStream_t stream, Op * op) {
	hipError_t err = hipModuleLaunchKernel(fn, cfg->gridDimX, cfg->gridDimY, cfg->gridDimZ,
											cfg->blockDimX, cfg->blockDimY, cfg->blockDimZ,
											cfg->sharedMemBytes, stream, op->op_args, NULL);
	if (err != hipSuccess) {
		fprintf(stderr, "hip backend: hipModuleLaunchKernel returned %s\n", hipGetErrorString(err));
		return -1;
	}
	return 0;
}

static int hip_submit_op(Dataflow_Handle * dataflow_handle, Op * op, int stream_id) {
	const char * nick = op->op_skeleton.header.op_nickname;
	hipStream_t stream;
	if (resolve_stream(dataflow_handle, stream_id, &stream, nick)) {
		return -1;
	}

	Hip_Function * f = NULL;
	long ind = find_table(&dataflow_handle->op_table, op->op_skeleton.identifier.fingerprint, false, (void **) &f);
	if (ind == -1 || !f) {
		fprintf(stderr, "Error: failed to find op with nickname %s and matching dtypes...\n", nick);
		return -1;
	}

	if (f->is_native) {
		Hip_Launch_Config cfg;
		memset(&cfg, 0, sizeof(cfg));
		if (f->set_launch_config(&cfg, dataflow_handle, f, op)) {
			fprintf(stderr, "hip backend: op %s: the launch configuration rejected these arguments\n", nick);
			return -1;
		}
		/* a zero-sized grid means there is no work (e.g. zero rows) */
		if (cfg.gridDimX == 0 || cfg.gridDimY == 0 || cfg.gridDimZ == 0) {
			return 0;
		}
		Hip_Context * hc = (Hip_Context *) dataflow_handle->ctx;
		if (f->function_config.shares_module_scratch && hc->two_pass_stream != HIP_NO_STREAM && hc->two_pass_stream != stream_id) {
			/* the previous op using the module scratch ran on another stream:
			 * wait for that stream's queued work */
			hipStream_t prev;
			if (resolve_stream(dataflow_handle, hc->two_pass_stream, &prev, nick)) {
				return -1;
			}
			HIP_CHECK_RET(hipEventRecord(hc->two_pass_event, prev), -1, "ordering op %s after the previous scratch user", nick);
			HIP_CHECK_RET(hipStreamWaitEvent(stream, hc->two_pass_event, 0), -1, "ordering op %s after the previous scratch user", nick);
		}
		if (launch(f->function_handle, &cfg, stream, op)) {
			fprintf(stderr, "hip backend: op %s: kernel launch failed\n", nick);
			return -1;
		}
		if (f->function_config.shares_module_scratch) {
			hc->two_pass_stream = stream_id;
		}
		if (f->finish_function_handle) {
			Hip_Launch_Config fcfg;
			memset(&fcfg, 0, sizeof(fcfg));
			if (f->set_finish_launch_config(&fcfg, dataflow_handle, f, op)) {
				fprintf(stderr, "hip backend: op %s: the second kernel's launch configuration rejected these arguments\n", nick);
				return -1;
			}
			if (fcfg.gridDimX && fcfg.gridDimY && fcfg.gridDimZ && launch(f->finish_function_handle, &fcfg, stream, op)) {
				fprintf(stderr, "hip backend: op %s: second kernel launch failed\n", nick);
				return -1;
			}
		}
		return 0;
	}

	if (!f->hip_external_func) {
		fprintf(stderr, "hip backend: op %s is registered as external but has no function to call\n", nick);
		return -1;
	}
	if (f->hip_external_func(dataflow_handle, stream_id, op, f->op_extra)) {
		fprintf(stderr, "hip backend: external op %s reported an error\n", nick);
		return -1;
	}
	return 0;
}

static int hip_submit_host_op(Dataflow_Handle * dataflow_handle, void * host_func, void * host_func_arg, int stream_id) {
	hipStream_t stream;
	if (resolve_stream(dataflow_handle, stream_id, &stream, "host op")) {
		return -1;
	}
	HIP_CHECK_RET(hipLaunchHostFunc(stream, (hipHostFn_t) host_func, host_func_arg), -1, "host function on stream");
	return 0;
}

/* ---------- 2. dependencies ---------- */

static void * hip_get_stream_state(Dataflow_Handle * dataflow_handle, int stream_id) {
	if (stream_id < 0 || stream_id >= dataflow_handle->num_streams) {
		fprintf(stderr, "hip backend: no stream state for stream id %d (the handle has %d streams)\n", stream_id, dataflow_handle->num_streams);
		return NULL;
	}
	hipStream_t stream = ((hipStream_t *) dataflow_handle->streams)[stream_id];
	hipEvent_t * events = (hipEvent_t *) dataflow_handle->stream_states;
	HIP_CHECK_RET(hipEventRecord(events[stream_id], stream), NULL, "recording the stream-state event");
	return &events[stream_id];
}

static int hip_submit_dependency(Dataflow_Handle * dataflow_handle, int stream_id, void * other_stream_state) {
	hipStream_t stream;
	if (!other_stream_state || resolve_stream(dataflow_handle, stream_id, &stream, "dependency")) {
		return -1;
	}
	HIP_CHECK_RET(hipStreamWaitEvent(stream, *((hipEvent_t *) other_stream_state), 0), -1,
					"making the stream wait for the given state");
	return 0;
}

static int hip_sync_stream(Dataflow_Handle * dataflow_handle, int stream_id) {
	hipStream_t stream;
	if (resolve_stream(dataflow_handle, stream_id, &stream, "sync")) {
		return -1;
	}
	HIP_CHECK_RET(hipStreamSynchronize(stream), -1, "synchronizing the stream");
	return 0;
}

static int hip_sync_handle(Dataflow_Handle * dataflow_handle) {
	HIP_CHECK_RET(hipSetDevice(dataflow_handle->device_id), -1, "device %d", dataflow_handle->device_id);
	HIP_CHECK_RET(hipDeviceSynchronize(), -1, "synchronizing handle (ctx id %d) on device %d", dataflow_handle->ctx_id, dataflow_handle->device_id);
	return 0;
}

/* ---------- 3. memory ---------- */

static void * hip_alloc_mem(Dataflow_Handle * dataflow_handle, uint64_t size_bytes) {
	void * p = NULL;
	HIP_CHECK_RET(hipSetDevice(dataflow_handle->device_id), NULL, "device %d", dataflow_handle->device_id);
	HIP_CHECK_RET(hipMalloc(&p, (size_t) size_bytes), NULL, "allocating %lu bytes on device %d",
					(unsigned long) size_bytes, dataflow_handle->device_id);
	return p;
}

static void hip_free_mem(Dataflow_Handle * dataflow_handle, void * dev_ptr) {
	if (hipSetDevice(dataflow_handle->device_id) != hipSuccess || hipFree(dev_ptr) != hipSuccess) {
		fprintf(stderr, "hip backend: releasing device memory %p on device %d failed\n", dev_ptr, dataflow_handle->device_id);
	}
}

static int hip_set_mem(Dataflow_Handle * dataflow_handle, int stream_id, void * dev_ptr, uint8_t val, uint64_t size_bytes) {
	if (stream_id == -1) {
		HIP_CHECK_RET(hipSetDevice(dataflow_handle->device_id), -1, "device %d", dataflow_handle->device_id);
		HIP_CHECK_RET(hipMemset(dev_ptr, val, (size_t) size_bytes), -1, "filling %lu bytes at %p",
						(unsigned long) size_bytes, dev_ptr);
		/* hipMemset on device memory may return before the fill is done, and
		 * the handle's streams do not wait for the null stream */
		HIP_CHECK_RET(hipStreamSynchronize(0), -1, "filling %lu bytes at %p", (unsigned long) size_bytes, dev_ptr);
		return 0;
	}
	hipStream_t stream;
	if (resolve_stream(dataflow_handle, stream_id, &stream, "set mem")) {
		return -1;
	}
	HIP_CHECK_RET(hipMemsetAsync(dev_ptr, val, (size_t) size_bytes, stream), -1, "filling %lu bytes at %p",
					(unsigned long) size_bytes, dev_ptr);
	return 0;
}

static int hip_enable_access_to_host_mem(Dataflow_Handle * dataflow_handle, void * host_ptr, uint64_t size_bytes, unsigned int flags) {
	HIP_CHECK_RET(hipHostRegister(host_ptr, (size_t) size_bytes, flags), -1,
					"registering host memory %p (%lu bytes, flags %u) for device %d",
					host_ptr, (unsigned long) size_bytes, flags, dataflow_handle->device_id);
	return 0;
}

static int hip_disable_access_to_host_mem(Dataflow_Handle * dataflow_handle, void * host_ptr) {
	HIP_CHECK_RET(hipHostUnregister(host_ptr), -1, "unregistering host memory %p for device %d",
					host_ptr, dataflow_handle->device_id);
	return 0;
}

static int hip_enable_access_to_peer_mem(Dataflow_Handle * dataflow_handle, Dataflow_Handle * peer_dataflow_handle) {
	if (peer_dataflow_handle->compute_type != dataflow_handle->compute_type) {
		fprintf(stderr, "hip backend: peer access needs two handles of the same compute type\n");
		return -1;
	}
	HIP_CHECK_RET(hipSetDevice(dataflow_handle->device_id), -1, "device %d", dataflow_handle->device_id);
	HIP_CHECK_RET(hipDeviceEnablePeerAccess(peer_dataflow_handle->device_id, 0), -1,
					"enabling access from device %d to device %d",
					dataflow_handle->device_id, peer_dataflow_handle->device_id);
	return 0;
}

static int hip_disable_access_to_peer_mem(Dataflow_Handle * dataflow_handle, Dataflow_Handle * peer_dataflow_handle) {
	if (peer_dataflow_handle->compute_type != dataflow_handle->compute_type) {
		fprintf(stderr, "hip backend: peer access needs two handles of the same compute type\n");
		return -1;
	}
	HIP_CHECK_RET(hipSetDevice(dataflow_handle->device_id), -1, "device %d", dataflow_handle->device_id);
	HIP_CHECK_RET(hipDeviceDisablePeerAccess(peer_dataflow_handle->device_id), -1,
					"disabling access from device %d to device %d",
					dataflow_handle->device_id, peer_dataflow_handle->device_id);
	return 0;
}

/* ---------- 4. transfers ---------- */

static int transfer(Dataflow_Handle * h, int stream_id, void * dst, const void * src, uint64_t n, hipMemcpyKind kind, const char * what) {
	if (stream_id == -1) {
		HIP_CHECK_RET(hipSetDevice(h->device_id), -1, "device %d", h->device_id);
		HIP_CHECK_RET(hipMemcpy(dst, src, (size_t) n, kind), -1, "%s of %lu bytes", what, (unsigned long) n);
		/* a device-to-device hipMemcpy may return before the copy is done,
		 * and the handle's streams do not wait for the null stream: finish
		 * it here, so the transfer is blocking as stream -1 promises */
		if (kind == hipMemcpyDeviceToDevice) {
			HIP_CHECK_RET(hipStreamSynchronize(0), -1, "%s of %lu bytes", what, (unsigned long) n);
		}
		return 0;
	}
	hipStream_t stream;
	if (resolve_stream(h, stream_id, &stream, what)) {
		return -1;
	}
	HIP_CHECK_RET(hipMemcpyAsync(dst, src, (size_t) n, kind, stream), -1, "%s of %lu bytes", what, (unsigned long) n);
	return 0;
}

static int hip_submit_inbound_transfer(Dataflow_Handle * dataflow_handle, int stream_id, void * dev_dest, void * host_src, uint64_t size_bytes) {
	return transfer(dataflow_handle, stream_id, dev_dest, host_src, size_bytes, hipMemcpyHostToDevice, "inbound transfer");
}

static int hip_submit_outbound_transfer(Dataflow_Handle * dataflow_handle, int stream_id, void * host_dest, void * dev_src, uint64_t size_bytes) {
	return transfer(dataflow_handle, stream_id, host_dest, dev_src, size_bytes, hipMemcpyDeviceToHost, "outbound transfer");
}

static int hip_submit_peer_transfer(Dataflow_Handle * dataflow_handle, int stream_id, void * dev_dest, void * dev_src, uint64_t size_bytes) {
	return transfer(dataflow_handle, stream_id, dev_dest, dev_src, size_bytes, hipMemcpyDeviceToDevice, "peer transfer");
}

/* ---------- init / destroy ---------- */

static int hip_set_device_info(Hip_Device_Info * info, int device_id) {
	hipDeviceProp_t prop;
	HIP_CHECK_RET(hipGetDeviceProperties(&prop, device_id), -1, "device %d", device_id);
	memset(info, 0, sizeof(*info));
	info->total_mem = prop.totalGlobalMem;
	info->cu_count = prop.multiProcessorCount;
	info->max_threads_per_block = MY_MIN(prop.maxThreadsPerBlock, HIP_DEV_UPPER_BOUND_MAX_THREADS_ALL_FUNC);
	info->max_smem_per_block = (int) prop.sharedMemPerBlock;
	info->optin_max_smem_per_block = (int) prop.sharedMemPerBlock;
	info->warp_size = prop.warpSize;
	info->l2_bytes = prop.l2CacheSize;
	strncpy(info->arch_name, prop.gcnArchName, sizeof(info->arch_name) - 1);
	info->arch_name[sizeof(info->arch_name) - 1] = '\0';
	/* "gfx950:sramecc+:xnack-" -> 950 (hex digits in the stepping, e.g. 90a, keep decimal prefix) */
	info->arch_num = 0;
	if (strncmp(prop.gcnArchName, "gfx", 3) == 0) {
		info->arch_num = (int) strtol(prop.gcnArchName + 3, NULL, 10);
	}
	int v = 0;
	info->num_xcds = (hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, device_id) == hipSuccess && v > 0) ? v : 1;
	v = -1;
	info->host_numa_id = (hipDeviceGetAttribute(&v, hipDeviceAttributeHostNumaId, device_id) == hipSuccess) ? v : -1;
	(void) hipGetLastError();
	return 0;
}

/* a failed initialisation releases what it had created (destroy handles the
 * fields that are still NULL) and reports -1 */
static int init_fail(Dataflow_Handle * dataflow_handle) {
	destroy_hip_dataflow_handle(dataflow_handle);
	return -1;
}

int init_hip_dataflow_handle(Dataflow_Handle * dataflow_handle, ComputeType compute_type, int device_id,
								int ctx_id, unsigned int ctx_flags,
								int num_streams, int * opt_stream_prios, char ** opt_stream_names) {
	(void) ctx_flags;
	if (num_streams < 0 || num_streams > MAX_STREAMS) {
		fprintf(stderr, "hip backend: num_streams must lie in [0, %d], got %d\n", MAX_STREAMS, num_streams);
		return -1;
	}
	memset(dataflow_handle, 0, sizeof(*dataflow_handle));
	dataflow_handle->compute_type = compute_type;
	dataflow_handle->device_id = device_id;
	dataflow_handle->ctx_id = ctx_id;

	int count = 0;
	HIP_CHECK_RET(hipGetDeviceCount(&count), -1, "counting devices");
	if (device_id < 0 || device_id >= count) {
		fprintf(stderr, "hip backend: device %d does not exist (%d devices visible)\n", device_id, count);
		return -1;
	}
	HIP_CHECK_RET(hipSetDevice(device_id), -1, "device %d", device_id);

	dataflow_handle->device_handle = malloc(sizeof(int));
	dataflow_handle->device_info = malloc(sizeof(Hip_Device_Info));
	dataflow_handle->ctx = calloc(1, sizeof(Hip_Context));
	if (!dataflow_handle->device_handle || !dataflow_handle->device_info || !dataflow_handle->ctx) {
		fprintf(stderr, "hip backend: out of host memory while creating the handle\n");
		return init_fail(dataflow_handle);
	}
	*((int *) dataflow_handle->device_handle) = device_id;
	Hip_Context * hc = (Hip_Context *) dataflow_handle->ctx;
	hc->device_id = device_id;
	hc->two_pass_stream = HIP_NO_STREAM;
	HIP_CHECK_RET(hipEventCreateWithFlags(&hc->two_pass_event, hipEventDisableTiming), init_fail(dataflow_handle), "creating the cross-stream ordering event on device %d", device_id);
	if (hip_set_device_info((Hip_Device_Info *) dataflow_handle->device_info, device_id)) {
		fprintf(stderr, "hip backend: reading the properties of device %d failed\n", device_id);
		return init_fail(dataflow_handle);
	}

	dataflow_handle->num_streams = num_streams;
	bool warned = false;
	for (int i = 0; i < MAX_STREAMS; i++) {
		dataflow_handle->stream_prios[i] = (i < num_streams) ? (opt_stream_prios ? opt_stream_prios[i] : HIP_DEFAULT_STREAM_PRIO) : -1;
		if (i < num_streams && dataflow_handle->stream_prios[i] != HIP_DEFAULT_STREAM_PRIO && !warned) {
			fprintf(stderr, "hip backend: warning: stream priorities are recorded, but every stream runs at the default priority\n");
			warned = true;
		}
		dataflow_handle->stream_names[i] = NULL;
		if (i < num_streams && opt_stream_names && opt_stream_names[i]) {
			dataflow_handle->stream_names[i] = strdup(opt_stream_names[i]);
			if (!dataflow_handle->stream_names[i]) {
				fprintf(stderr, "hip backend: out of host memory for a stream name\n");
				return init_fail(dataflow_handle);
			}
		}
	}

	size_t ns = (size_t) (num_streams > 0 ? num_streams : 1);
	dataflow_handle->streams = calloc(ns, sizeof(hipStream_t));
	dataflow_handle->stream_states = calloc(ns, sizeof(hipEvent_t));
	if (!dataflow_handle->streams || !dataflow_handle->stream_states) {
		fprintf(stderr, "hip backend: out of host memory for the stream tables\n");
		return init_fail(dataflow_handle);
	}
	hipStream_t * streams = (hipStream_t *) dataflow_handle->streams;
	hipEvent_t * events = (hipEvent_t *) dataflow_handle->stream_states;
	for (int i = 0; i < num_streams; i++) {
		HIP_CHECK_RET(hipStreamCreateWithFlags(&streams[i], hipStreamNonBlocking), init_fail(dataflow_handle), "creating stream %d on device %d", i, device_id);
		HIP_CHECK_RET(hipEventCreateWithFlags(&events[i], hipEventDisableTiming), init_fail(dataflow_handle), "creating the state event of stream %d on device %d", i, device_id);
	}

	dataflow_handle->num_native_function_libs = 0;
	dataflow_handle->num_ops = 0;
	if (init_table(&dataflow_handle->op_table, hip_op_table_hash_func, OP_IDENTIFIER_FINGERPRINT_NUM_BYTES, sizeof(Hip_Function),
					OP_TABLE_MIN_SIZE, OP_TABLE_MAX_SIZE, 1.0f, 1.0f)) {
		fprintf(stderr, "hip backend: the op table could not be created\n");
		return init_fail(dataflow_handle);
	}

	dataflow_handle->register_native_code = hip_register_native_code;
	dataflow_handle->register_external_code = hip_register_external_code;
	dataflow_handle->submit_op = hip_submit_op;
	dataflow_handle->submit_host_op = hip_submit_host_op;
	dataflow_handle->get_stream_state = hip_get_stream_state;
	dataflow_handle->submit_dependency = hip_submit_dependency;
	dataflow_handle->sync_stream = hip_sync_stream;
	dataflow_handle->sync_handle = hip_sync_handle;
	dataflow_handle->alloc_mem = hip_alloc_mem;
	dataflow_handle->free_mem = hip_free_mem;
	dataflow_handle->set_mem = hip_set_mem;
	dataflow_handle->enable_access_to_host_mem = hip_enable_access_to_host_mem;
	dataflow_handle->disable_access_to_host_mem = hip_disable_access_to_host_mem;
	dataflow_handle->enable_access_to_peer_mem = hip_enable_access_to_peer_mem;
	dataflow_handle->disable_access_to_peer_mem = hip_disable_access_to_peer_mem;
	dataflow_handle->submit_inbound_transfer = hip_submit_inbound_transfer;
	dataflow_handle->submit_outbound_transfer = hip_submit_outbound_transfer;
	dataflow_handle->submit_peer_transfer = hip_submit_peer_transfer;
	return 0;
}

int destroy_hip_dataflow_handle(Dataflow_Handle * dataflow_handle) {
	int ret = 0;
	if (hipSetDevice(dataflow_handle->device_id) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
		ret = -1;
	}
	hipStream_t * streams = (hipStream_t *) dataflow_handle->streams;
	hipEvent_t * events = (hipEvent_t *) dataflow_handle->stream_states;
	for (int i = 0; i < dataflow_handle->num_streams; i++) {
		if (events && events[i]) hipEventDestroy(events[i]);
		if (streams && streams[i]) hipStreamDestroy(streams[i]);
		free(dataflow_handle->stream_names[i]);
		dataflow_handle->stream_names[i] = NULL;
	}
	for (int i = 0; i < dataflow_handle->num_native_function_libs; i++) {
		hipModule_t * m = (hipModule_t *) dataflow_handle->native_function_libs[i];
		if (m) {
			hipModuleUnload(*m);
			free(m);
		}
		dataflow_handle->native_function_libs[i] = NULL;
	}
	dataflow_handle->num_native_function_libs = 0;
	destroy_table(&dataflow_handle->op_table);
	free(dataflow_handle->streams);
	free(dataflow_handle->stream_states);
	free(dataflow_handle->device_handle);
	free(dataflow_handle->device_info);
	Hip_Context * hc = (Hip_Context *) dataflow_handle->ctx;
	if (hc && hc->two_pass_event) hipEventDestroy(hc->two_pass_event);
	free(dataflow_handle->ctx);
	dataflow_handle->streams = NULL;
	dataflow_handle->stream_states = NULL;
	dataflow_handle->device_handle = NULL;
	dataflow_handle->device_info = NULL;
	dataflow_handle->ctx = NULL;
	dataflow_handle->num_streams = 0;
	dataflow_handle->num_ops = 0;
	return ret;
}

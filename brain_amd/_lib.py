"""ctypes binding of libbrain_hip.so (the C ABI declared in include/brain_hip.h).

There is no fallback: if the HIP library is missing this module raises, so a
caller can never silently run some other implementation.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbrain_hip.so")

BH_OK, BH_ERR_INVALID, BH_ERR_HIP, BH_ERR_UNSUPPORTED, BH_ERR_NOMEM, BH_ERR_TIMEOUT = 0, -1, -2, -3, -4, -5
BH_OUT_F32, BH_OUT_BF16, BH_OUT_I32 = 0, 1, 2
BH_CREATE_LENIENT = 1
BH_VARIANT_PACKED_INT8, BH_VARIANT_WORKGROUP_PER_OUTPUT = 1, 2


class BrainHipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class CapsT(C.Structure):
    _fields_ = [
        ("compute_units", C.c_uint32), ("max_workgroup_size", C.c_uint32),
        ("workgroup_mem_bytes", C.c_uint32), ("subgroup_size", C.c_uint32),
        ("unified_memory", C.c_uint32), ("workgroup_reductions", C.c_uint32),
        ("peak_bandwidth_gbs", C.c_float), ("peak_gflops", C.c_float),
        ("numeric_f32", C.c_uint32), ("numeric_int8_dot", C.c_uint32),
        ("numeric_f16", C.c_uint32), ("numeric_bf16", C.c_uint32),
        ("numeric_f16_storage", C.c_uint32), ("numeric_bf16_storage", C.c_uint32),
        ("numeric_coop_matrix", C.c_uint32),
        ("max_buffer_bytes", C.c_uint64), ("max_storage_binding_bytes", C.c_uint64),
        ("device_name", C.c_char * 64),
    ]


class KernelTimeT(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("ms", C.c_double), ("calls", C.c_uint64)]


class StatsT(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("submits", "dispatches", "readbacks", "bind_groups", "uniform_allocs")]


class Qwen3ConfigT(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("vocab", "n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim", "d_ff")] + \
               [("rope_theta", C.c_float), ("rms_eps", C.c_float), ("tie_embeddings", C.c_uint32), ("qk_norm", C.c_uint32),
                ("kv_int8", C.c_uint32), ("kv_block_size", C.c_uint32), ("kv_num_blocks", C.c_uint32)]


class CostT(C.Structure):
    _fields_ = [("flops", C.c_uint64), ("int_ops", C.c_uint64), ("bytes", C.c_uint64)]


vp, u32, u64, i32, f32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_float
P = C.POINTER
# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES = {
    "bh_last_error": (C.c_char_p, []),
    "bh_abi_version": (i32, []),
    "bh_max_abs_rows": (i32, [vp, vp, u32, u32, vp]),
    "bh_quant_pack": (i32, [vp, vp, vp, u32, u32, vp]),
    "bh_quantize_rows": (i32, [vp, vp, u32, u32, vp, vp]),
    "bh_quantize_rows_bf16": (i32, [vp, vp, u32, u32, vp, vp]),
    "bh_matmul_i8": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, u32, u32, u32]),
    "bh_matmul_i8_gemv": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, u32, u32, u32]),
    "bh_matmul_i8_dyn": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, u32, u32, u32]),
    "bh_matmul_i8_dyn_quant": (i32, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, vp, vp]),
    "bh_matmul_i8_dyn_noalloc": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, u32, u32, u32]),
    "bh_paged_kv_append_i8": (i32, [vp, vp, vp, vp, vp, vp, u64, vp, u64, u32, u32, u32, u32]),
    "bh_paged_decode_scores_i8": (i32, [vp, vp, vp, u64, vp, vp, vp, u64, vp] + [u32] * 8 + [f32]),
    "bh_paged_decode_apply_i8": (i32, [vp, vp, vp, u64, vp, vp, vp, u64, vp] + [u32] * 8),
    "bh_reserve_workspace": (i32, [vp, u32, u32, u32]),
    "bh_matmul_i8_static": (i32, [vp, vp, vp, f32, f32, vp, u32, u32, u32]),
    "bh_linear_i8": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, i32, u32, u32, u32]),
    "bh_quantize_weight_device": (i32, [vp, vp, u32, u32, vp, vp]),
    "bh_f32_to_bf16": (i32, [vp, vp, vp, C.c_uint64]),
    "bh_roof_mfma_i8": (i32, [vp, u32, u32, vp]),
    "bh_roof_hbm_read": (i32, [vp, vp, u64, u32, vp]),
    "bh_qwen3_create": (i32, [vp, u32, u32, u32, i32, vp]),
    "bh_qwen3_destroy": (None, [vp]),
    "bh_qwen3_set_weight": (i32, [vp, C.c_char_p, vp, u64]),
    "bh_qwen3_set_weight_i8": (i32, [vp, C.c_char_p, vp, vp, u32, u32]),
    "bh_qwen3_init_random": (i32, [vp, u64]),
    "bh_qwen3_prefill": (i32, [vp, vp, u32, u32, vp]),
    "bh_qwen3_decode": (i32, [vp, u32, u32, vp]),
    "bh_qwen3_logits": (i32, [vp, vp, u64]),
    "bh_qwen3_lengths": (i32, [vp, vp, u32]),
    "bh_qwen3_kv_read": (i32, [vp, u32, u32, u32, u32, u32, vp, vp]),
    "bh_qwen3_stream": (vp, [vp]),
    "bh_qwen3_load": (i32, [vp, C.c_char_p]),
    "bh_qwen3_set_kv_clip": (i32, [vp, u32, u32, vp]),
    "bh_qwen3_set_block_table": (i32, [vp, vp, u32, u32]),
    "bh_qwen3_kv_pool": (i32, [vp, u32, u32, P(vp), P(u64), P(vp), P(u64)]),
    "bh_qwen3_autotune": (i32, [vp, u32]),
    "bh_tune_i8": (i32, [vp, u32, u32, u32, u32, vp, vp]),
    "bh_tune_set": (i32, [u32, u32, u32, i32]),
    "bh_tune_get": (i32, [u32, u32, u32]),
    "bh_tune_clear": (None, []),
    "bh_tune_save": (i32, [C.c_char_p]),
    "bh_tune_load": (i32, [C.c_char_p]),
    "bh_st_describe": (i32, [C.c_char_p, C.c_char_p, vp, vp, u32, vp]),
    "bh_backend_create": (i32, [P(C.c_char_p), P(C.c_char_p), u32, i32, u32, P(vp)]),
    "bh_backend_destroy": (None, [vp]),
    "bh_backend_kind": (C.c_char_p, [vp]),
    "bh_kernel_index": (i32, [vp, C.c_char_p]),
    "bh_backend_stream": (vp, [vp]),
    "bh_caps": (i32, [vp, P(CapsT)]),
    "bh_storage": (i32, [vp, u64, P(vp)]),
    "bh_storage_init": (i32, [vp, C.c_char_p, vp, u64, P(vp)]),
    "bh_buffer_retain": (vp, [vp]),
    "bh_buffer_release": (None, [vp]),
    "bh_buffer_words": (u64, [vp]),
    "bh_buffer_device_ptr": (vp, [vp]),
    "bh_write": (i32, [vp, vp, vp, u64]),
    "bh_write_at": (i32, [vp, vp, u64, vp, u64]),
    "bh_read": (i32, [vp, vp, vp, u64]),
    "bh_step": (i32, [vp, u32, P(vp), u32, P(u32), u32, u32, P(vp)]),
    "bh_step_sliced": (i32, [vp, u32, P(vp), P(u64), u32, P(u32), u32, u32, P(vp)]),
    "bh_step_retain": (vp, [vp]),
    "bh_step_release": (None, [vp]),
    "bh_submit": (i32, [vp, P(vp), u32, P(vp), u32]),
    "bh_flush": (i32, [vp]),
    "bh_poll_wait": (i32, [vp]),
    "bh_poll_wait_timeout": (i32, [vp, u32]),
    "bh_set_kernel_timing": (i32, [vp, i32]),
    "bh_kernel_times": (i32, [vp, P(KernelTimeT), u32]),
    "bh_reset_kernel_times": (None, [vp]),
    "bh_stats": (i32, [vp, P(StatsT)]),
    "bh_quantize_weight": (i32, [vp, u64, u64, vp, vp]),
    "bh_quantize_weight_q4": (i32, [vp, u64, u64, vp, vp]),
    "bh_matmul_q4_gemv": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, u32, u32, u32]),
    "bh_matmul_q4_dyn": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, u32, u32, u32]),
    "bh_matmul_q4": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, u32, u32, u32]),
    "bh_moe_linear_gated_i8": (i32, [vp, vp, vp, vp, vp, vp, u32, u32, vp, u32, u32, u32]),
    "bh_dequantize_weight": (i32, [vp, vp, u64, u64, vp]),
    "bh_quant_rows_steps": (i32, [vp, P(u32), vp, vp, vp, u32, u32, u32, P(vp)]),
    "bh_mm8_rows_off": (i32, [vp, u32, vp, vp, vp, vp, vp, u32, u64, u32, u32, u32, P(vp)]),
    "bh_select_i8": (i32, [u32, u32, u32, i32, i32, P(i32)]),
    "bh_variant_kernel": (C.c_char_p, [i32]),
    "bh_cost": (i32, [C.c_char_p, P(u32), u32, P(CostT)]),
}

_lib = None


def load():
    """Load libbrain_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m brain_amd.build` "
                          "(or __graft_entry__.build()); there is no non-HIP fallback")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc):
    """Raise BrainHipError for a negative status."""
    if rc < 0:
        raise BrainHipError(rc, load().bh_last_error().decode())
    return rc

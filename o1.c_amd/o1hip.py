"""ctypes bindings of libo1hip.so (the C-ABI declared in include/*.h).

Mirrors the reference's host interface for the per-block forward path:
hd_linear / hd_sdpa_* / hd_decoder_block / hd_forward / hd_lora_merge_gpu
(reference: src/cuda/hd_cuda.h, gemm.h, include/hd_cudnn_sdpa.h,
src/model/block.h, forward.h, include/hd_lora.h). Tensors are torch device
tensors; only their data pointers cross the boundary.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libo1hip.so")

c_void_p, c_int, c_int64, c_float, c_size_t, c_char_p = (
    ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t, ctypes.c_char_p)

HD_OK, HD_ERR_MISSING, HD_ERR_OOM, HD_ERR_RUNTIME, HD_ERR_UNSUPPORTED = 0, 6, 7, 8, 9
HD_ERR_IO, HD_ERR_PARSE = 1, 2
HD_ERR_MISMATCH = 5


class hd_block_binding(ctypes.Structure):
    _fields_ = [("layer_idx", c_int)] + [(n, c_void_p) for n in (
        "q_proj", "k_proj", "v_proj", "o_proj", "input_ln", "post_ln", "gate_proj", "up_proj",
        "down_proj", "q_norm", "k_norm")]


class hd_block_internals(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("ln0", "attn_hidden", "attn_resid", "post_ln", "mlp_out")]


class hd_block_config(ctypes.Structure):
    _fields_ = [("eps", c_float), ("rope_theta", c_float), ("attention_scaling", c_float),
                ("section", c_int64 * 3), ("interleaved", c_int)]


class hd_device_alloc(ctypes.Structure):
    _fields_ = [("dev_ptr", c_void_p), ("nbytes", c_int64), ("name", ctypes.c_char * 256)]


class hd_weight_store(ctypes.Structure):
    _fields_ = [("device_id", c_int), ("device_name", ctypes.c_char * 256), ("compute_major", c_int),
                ("compute_minor", c_int), ("device_mem_bytes", c_int64), ("host_bytes_loaded", c_int64),
                ("device_bytes_allocated", c_int64), ("n_allocations", c_int64),
                ("largest_numel", c_int64), ("largest_name", ctypes.c_char * 256),
                ("allocs", ctypes.POINTER(hd_device_alloc)), ("n_allocs", c_int64), ("gemm", c_void_p),
                ("arena_ptr", c_void_p), ("arena_bytes", c_int64), ("upload_stream", c_void_p)]


class hd_gguf_tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 8),
                ("type", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


class hd_gguf_file(ctypes.Structure):
    _fields_ = [("path", ctypes.c_char_p), ("n_tensors", c_int64),
                ("tensors", ctypes.POINTER(hd_gguf_tensor)), ("alignment", ctypes.c_uint64),
                ("tensor_data_off", ctypes.c_uint64), ("payload_bytes", ctypes.c_uint64)] + [
                (n, ctypes.c_char_p) for n in ("arch", "name", "profile", "variant", "revision", "dtype",
                                               "quantization")] + [
                ("num_layers", c_int64), ("layout_version", c_int64)]


class hd_forward_binding(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in (
        "embed_tokens", "te0_w", "te0_b", "te2_w", "te2_b", "xe1_w", "xe2_w", "xe2_b", "fl_w",
        "fl_b", "fnorm_w")] + [("n_layers", c_int), ("blocks", ctypes.POINTER(hd_block_binding))]


class hd_forward_workspace(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in (
        "hidden_a", "hidden_b", "h_text", "norm_out", "head_out", "t_emb", "te_hidden", "freq",
        "freq_bf16", "t_scaled", "xe_stage", "xe_out", "xe_ref")] + [
        ("n_ref", c_int), ("block_scratch", c_void_p), ("block_scratch_bytes", c_int64),
        ("sdpa", c_void_p)]


class hd_forward_diagnostics(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in (
        "after_embedding", "after_timestep_conditioning", "after_target_embedding",
        "after_block_0_input", "after_block_0", "after_block_mid", "after_block_last",
        "before_final_norm", "after_final_norm", "after_final_head")]


class hd_torch_rng(ctypes.Structure):
    _fields_ = [("seed_", ctypes.c_uint64), ("left_", c_int), ("seeded_", c_int),
                ("next_", ctypes.c_uint32), ("state", ctypes.c_uint32 * 624)]


class hd_scheduler(ctypes.Structure):
    _fields_ = [("sigmas", c_float * 64), ("num_steps", c_int), ("step_index", c_int),
                ("noise_clip_std", c_float)]


class hd_scheduler_unipc(ctypes.Structure):
    _fields_ = [("model_outputs", c_void_p * 2), ("last_sample", c_void_p),
                ("has_last_sample", c_int), ("this_order", c_int), ("lower_order_nums", c_int),
                ("step_index", c_int)]


class hd_unipc_plan(ctypes.Structure):
    _fields_ = [("corr_order", c_int), ("pred_order", c_int), ("next_this_order", c_int),
                ("next_lower_order", c_int)] + [(n, ctypes.c_double) for n in (
                    "c_sig_t", "c_sig_s0", "c_alpha_t", "c_h_phi_1", "c_B_h", "c_rhos0", "c_rhos1",
                    "c_inv_rks0", "p_sig_t", "p_sig_s0", "p_alpha_t", "p_h_phi_1", "p_B_h",
                    "p_rhos_p", "p_inv_rks0")]


class hd_lora_entry(ctypes.Structure):
    _fields_ = [("lora_prefix", ctypes.c_char * 256), ("base_tensor", ctypes.c_char * 256),
                ("rank", ctypes.c_uint32), ("in_dim", ctypes.c_uint32),
                ("out_dim", ctypes.c_uint32), ("alpha", c_float), ("multiplier", c_float),
                ("down_dev", c_void_p), ("up_dev", c_void_p), ("base_dev", c_void_p)]


class hd_ref_geom(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("tokens", "grid_h", "grid_w", "cond_h", "cond_w")]


class hd_sequence(ctypes.Structure):
    _fields_ = [("input_ids", ctypes.POINTER(ctypes.c_int64)), ("pos_f32", ctypes.POINTER(c_float)),
                ("mask_bf16", ctypes.POINTER(ctypes.c_uint8)), ("vinput_mask", ctypes.POINTER(ctypes.c_uint8)),
                ("sec", ctypes.c_int64 * 3), ("text_len", c_int), ("image_len", c_int),
                ("img_begin", c_int), ("S", c_int), ("n_refs", c_int),
                ("ref_len", c_int * 20), ("ref_begin", c_int * 20)]


class hd_vision_block_binding(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "qkv_w", "qkv_b",
                                        "proj_w", "proj_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b")]


class hd_vision_merger_binding(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("norm_w", "norm_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b")]


class hd_vision_binding(ctypes.Structure):
    _fields_ = [("patch_proj_w", c_void_p), ("patch_proj_b", c_void_p), ("pos_embed", c_void_p),
                ("blocks", hd_vision_block_binding * 27), ("merger", hd_vision_merger_binding),
                ("deepstack", hd_vision_merger_binding * 3)]


VISION_WS_BUFFERS = ("patch_out", "pos_emb", "rot", "cosf", "sinf", "h_a", "h_b", "ln1", "qkv", "q",
                     "k", "v", "qr", "kr", "scores", "probs", "attn_out", "attn_resid", "ln2", "fc1",
                     "fc2", "mlp_resid", "merged", "merge_norm", "merge_fc1", "merge_fc2",
                     "ds_merged", "ds_fc1", "ds_fc2")


class hd_vision_workspace(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in VISION_WS_BUFFERS] + \
               [(n, c_void_p) for n in ("pos_idx", "pos_wgt", "rot_coords", "rot_inv", "tables")] + \
               [("tables_n", c_int), ("tables_gh", c_int), ("tables_gw", c_int),
                ("bytes", ctypes.c_int64), ("sdpa", c_void_p), ("block0_snap", c_void_p),
                ("block0_snaps", c_void_p * 16), ("block_out_snaps", c_void_p * 27),
                ("merger_snaps", c_void_p * 5), ("ds_merger_snaps", (c_void_p * 4) * 3)]


class hd_vision_offsets(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "patch_out", "pos_emb", "rot", "h_a", "h_b", "ln1", "attn_resid", "ln2", "fc2", "mlp_resid",
        "q", "k", "v", "qr", "kr", "qkv", "scores", "probs", "mask", "attn_out", "fc1", "cosf",
        "sinf", "merged", "merge_norm", "merge_fc1", "merge_fc2", "ds_merged", "ds_fc1", "ds_fc2",
        "total_bytes")]


class hd_visual_cond(ctypes.Structure):
    _fields_ = [("image_embeds", c_void_p), ("deepstack", c_void_p * 3), ("visual_mask", c_void_p),
                ("v_tokens", c_int)]


class hd_lora_spec(ctypes.Structure):
    _fields_ = [("path", ctypes.c_char_p), ("multiplier", c_float)]


class hd_lora_config(ctypes.Structure):
    _fields_ = [("items", ctypes.POINTER(hd_lora_spec)), ("count", c_size_t)]


P = c_void_p
# name -> (restype, argtypes); every symbol include/*.h declares.
SIGNATURES = {
    # hidream_hip.h
    "hd_last_error": (c_char_p, []),
    "hd_set_error": (None, [c_char_p]),
    # hd_hip.h
    "hd_bf16_to_f32": (c_float, [ctypes.c_uint16]),
    "hd_f32_to_bf16": (ctypes.c_uint16, [c_float]),
    "hd_bf16_buf_to_f32": (None, [P, P, c_size_t]),
    "hd_f32_buf_to_bf16": (None, [P, P, c_size_t]),
    "hd_cuda_last_error": (c_char_p, []),
    "hd_cuda_clear_error": (None, []),
    "hd_hip_set_stream": (None, [P]),
    "hd_hip_get_stream": (P, []),
    "hd_hip_sync": (c_int, []),
    "hd_rmsnorm": (None, [P, P, P, c_int, c_int, c_float]),
    "hd_silu": (None, [P, P, c_size_t]),
    "hd_swiglu": (None, [P, P, P, c_size_t]),
    "hd_residual_add": (None, [P, P, P, c_size_t]),
    "hd_linear": (None, [P, P, P, P, c_int, c_int, c_int, c_int]),
    "hd_timestep_embed": (None, [P, P, c_int, c_int]),
    "hd_mrope_cos_sin": (None, [P, c_int, c_int, P, c_int, c_int, c_float, c_float, c_int, P, P]),
    "hd_apply_rotary": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_apply_rotary_f32": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_attention_eager": (None, [P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_float]),
    "hd_head_split": (None, [P, P, c_int, c_int, c_int]),
    "hd_head_merge": (None, [P, P, c_int, c_int, c_int]),
    "hd_gather_rows": (None, [P, P, P, c_int, c_int, c_int64]),
    "hd_apply_tms_condition": (None, [P, P, P, P, c_int, c_int, c_int64]),
    "hd_scale_f32": (None, [P, P, c_float, c_int]),
    "hd_f32_convert_bf16": (None, [P, P, c_int]),
    "hd_sched_bf16_upcast": (None, [P, P, c_int]),
    "hd_sched_denoised": (None, [P, P, c_float, P, c_int]),
    "hd_sched_z_next": (None, [P, P, c_float, c_float, P, c_int]),
    "hd_sched_vcond": (None, [P, P, c_float, P, c_int]),
    "hd_sched_flow_match_step": (None, [P, P, c_float, c_float, P, c_int]),
    "hd_sched_cfg_guided": (None, [P, P, c_float, P, c_int]),
    "hd_add_rmsnorm": (None, [P, P, P, P, P, c_int, c_int, c_float]),
    "hd_rope_table": (None, [P, c_int, P, c_int, c_int, c_float, c_float, c_int, P]),
    "hd_rope_table_dev": (None, [P, c_int, P, c_int, c_int, c_float, c_float, c_int, P]),
    "hd_qkv_epilogue": (None, [P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float]),
    "hd_transpose_sd": (None, [P, P, c_int, c_int, c_int]),
    "hd_patchify_f32": (None, [P, P, c_int, c_int, c_int, c_int]),
    "hd_unpatchify_f32": (None, [P, P, c_int, c_int, c_int, c_int]),
    "hd_patchify_bf16": (None, [P, P, c_int, c_int, c_int, c_int]),
    # hd_gemm.h
    "hd_gemm_runtime_init": (P, [c_int, c_size_t]),
    "hd_gemm_runtime_destroy": (None, [P]),
    "hd_gemm_workspace": (P, [P]),
    "hd_gemm_workspace_bytes": (c_size_t, [P]),
    "hd_linear_reference": (None, [P, P, P, P, c_int, c_int, c_int, c_int]),
    "hd_gemm_set_backend": (None, [c_int]),
    "hd_gemm_set_prod_backend": (None, [c_int]),
    "hd_linear_residual": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_linear_swiglu": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_linear_swiglu_ws": (None, [P, P, P, P, c_int, c_int, c_int, P, ctypes.c_int64]),
    "hd_linear_concat3": (None, [P, P, c_int, P, c_int, P, c_int, P, c_int, c_int]),
    "hd_gemm_config_name": (c_char_p, [c_int, c_int, c_int, c_int]),
    "hd_mfma_probe": (ctypes.c_double, [P, c_int, c_int, c_int, c_int, P]),
    "hd_tokenizer_load": (c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p]),
    "hd_tokenizer_unload": (None, []),
    "hd_tokenizer_encode": (c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.POINTER(c_int)), ctypes.POINTER(c_size_t)]),
    "hd_tokenizer_encode_prompt": (c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.POINTER(c_int)), ctypes.POINTER(c_size_t)]),
    "hd_tokenizer_build_template": (c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]),
    "hd_tokenizer_build_ref_template": (c_int, [ctypes.c_char_p, c_int, ctypes.POINTER(ctypes.c_void_p)]),
    "hd_tokenizer_special_id": (c_int, [ctypes.c_char_p]),
    "hd_tokenizer_free_ids": (None, [ctypes.POINTER(c_int)]),
    "hd_linear_qkv_rope": (c_int, [P, P, P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float]),
    "hd_linear_qkv_rope_ws": (c_int, [P] * 10 + [c_int] * 5 + [c_float, P, ctypes.c_int64]),
    # hd_sdpa.h
    "hd_sdpa_create": (c_int, [ctypes.POINTER(c_void_p), c_int, c_int, c_int, c_int, c_int, c_int, c_float]),
    "hd_sdpa_execute": (c_int, [P, P, P, P, P, P, P]),
    "hd_sdpa_destroy": (None, [P]),
    "hd_sdpa_create_split": (c_int, [ctypes.POINTER(c_void_p), c_int, c_int, c_int, c_int, c_int, c_int, c_float]),
    "hd_sdpa_execute_split": (c_int, [P, P, P, P, P, P]),
    "hd_sdpa_execute_split_pass": (c_int, [P, c_int, P, P, P, P, P]),
    "hd_sdpa_plan_stage": (P, [P]),
    "hd_sdpa_create_prod": (c_int, [ctypes.POINTER(c_void_p), c_int, c_int, c_int, c_int, c_int, c_int, c_float]),
    "hd_flash_attention": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int]),
    "hd_sdpa_plan_ar_len": (c_int, [P]),
    "hd_flash_attention_ws": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int,
                                      P, c_int64]),
    "hd_flash_ws_bytes": (c_int64, []),
    "hd_flash_vt_bytes": (c_int64, [c_int, c_int, c_int]),
    "hd_flash_make_vt": (None, [P, P, c_int, c_int]),
    # hd_weights.h
    "hd_weight_store_find": (P, [ctypes.POINTER(hd_weight_store), c_char_p]),
    "hd_device_info": (c_int, [c_int, ctypes.POINTER(hd_weight_store)]),
    "hd_weights_to_device_gguf": (c_int, [c_char_p, c_int, ctypes.POINTER(hd_weight_store)]),
    "hd_weight_store_free": (None, [ctypes.POINTER(hd_weight_store)]),
    "hd_weights_last_error": (c_char_p, []),
    "hd_gguf_open": (c_int, [c_char_p, ctypes.POINTER(hd_gguf_file)]),
    "hd_gguf_close": (None, [ctypes.POINTER(hd_gguf_file)]),
    "hd_gguf_read_tensor": (c_int, [ctypes.POINTER(hd_gguf_file), ctypes.POINTER(hd_gguf_tensor), P]),
    "hd_gguf_last_error": (c_char_p, []),
    # hd_block.h
    "hd_block_get_config": (None, [ctypes.POINTER(hd_block_config)]),
    "hd_block_set_config": (None, [ctypes.POINTER(hd_block_config)]),
    "hd_decoder_block_scratch_bytes": (c_int64, [c_int64, c_int, c_int, c_int, c_int, c_int]),
    "hd_block_resolve": (c_int, [ctypes.POINTER(hd_weight_store), c_int, ctypes.POINTER(hd_block_binding)]),
    "hd_decoder_block": (c_int, [P, P, P, ctypes.POINTER(hd_block_binding), P, P, c_int64,
                                 ctypes.POINTER(hd_block_internals), P, c_int64, c_int, c_int,
                                 c_int, c_int, c_int, P]),
    "hd_decoder_block_batched_scratch_bytes": (c_int64, [c_int, c_int64, c_int, c_int, c_int, c_int, c_int]),
    "hd_decoder_block_batched": (c_int, [P, P, P, c_int, ctypes.POINTER(hd_block_binding), P,
                                         c_int64, ctypes.POINTER(hd_block_internals), P, c_int,
                                         c_int64, c_int, c_int, c_int, c_int, c_int]),
    # hd_forward.h
    "hd_forward_resolve": (c_int, [ctypes.POINTER(hd_weight_store), c_int, ctypes.POINTER(hd_forward_binding)]),
    "hd_forward_binding_free": (None, [ctypes.POINTER(hd_forward_binding)]),
    "hd_forward_workspace_bytes": (c_int64, [c_int64, c_int, c_int, c_int, c_int, c_int, c_int, ctypes.POINTER(c_int64)]),
    "hd_forward": (c_int, [ctypes.POINTER(hd_forward_binding), ctypes.POINTER(hd_forward_workspace),
                           P, c_int, P, P, P, c_int, P, P, P, c_int, c_int, c_int, c_int, c_int,
                           c_int, c_int, ctypes.POINTER(hd_forward_diagnostics), P, P]),
    "hd_forward_num_layers": (c_int, [ctypes.POINTER(hd_forward_binding)]),
    "hd_forward_ws_offset": (c_int64, [c_char_p, c_int64, c_int, c_int, c_int, c_int, c_int, c_int, c_int, ctypes.POINTER(c_int64)]),
    "hd_forward_batched_workspace_bytes": (c_int64, [c_int, c_int64, c_int, c_int, c_int, c_int, c_int, c_int]),
    "hd_forward_batched": (c_int, [ctypes.POINTER(hd_forward_binding), ctypes.POINTER(hd_forward_workspace),
                                   c_int, P, c_int, P, c_int, P, c_int, P, c_int, c_int, c_int,
                                   c_int, c_int, c_int, c_int, ctypes.POINTER(hd_forward_diagnostics), P, P]),
    # hd_lora.h
    "hd_lora_merge_gpu": (c_int, [ctypes.POINTER(hd_lora_entry), c_size_t, P]),
    "hd_lora_apply": (c_int, [ctypes.POINTER(hd_lora_config), ctypes.POINTER(hd_weight_store), c_int]),
    "hd_lora_last_error": (c_char_p, []),
    # hd_host.h
    "hd_torch_rng_seed": (None, [ctypes.POINTER(hd_torch_rng), ctypes.c_uint64]),
    "hd_torch_rng_u32": (ctypes.c_uint32, [ctypes.POINTER(hd_torch_rng)]),
    "hd_torch_uniform_f32": (c_float, [ctypes.POINTER(hd_torch_rng)]),
    "hd_torch_randn_f32": (None, [ctypes.POINTER(hd_torch_rng), P, c_int64]),
    "hd_scheduler_init": (c_int, [ctypes.POINTER(hd_scheduler), P, c_int, c_float]),
    "hd_scheduler_sigma": (c_float, [ctypes.POINTER(hd_scheduler)]),
    "hd_scheduler_derive_dev": (c_int, [ctypes.POINTER(hd_scheduler), c_float]),
    "hd_scheduler_derive_flash": (c_int, [ctypes.POINTER(hd_scheduler), c_int, c_float, c_float]),
    "hd_scheduler_derive_flow_match": (c_int, [ctypes.POINTER(hd_scheduler), c_int, c_float, c_float]),
    "hd_scheduler_derive_default": (c_int, [ctypes.POINTER(hd_scheduler), c_int, c_float, c_float]),
    "hd_scheduler_noise_scale": (c_float, [ctypes.POINTER(hd_scheduler), c_int, c_float, c_float]),
    "hd_scheduler_step": (c_int, [ctypes.POINTER(hd_scheduler), P, P, P, c_float, P, c_int, P]),
    "hd_seq_t2i_positions": (c_int, [c_int, c_int, c_int, c_int, P]),
    "hd_seq_t2i_mask": (c_int, [c_int, c_int, P]),
    "hd_seq_grid_positions": (c_int, [c_int, c_int, P, P, P, P, c_float, P]),
    "hd_initial_noise": (None, [ctypes.c_uint64, c_int, c_int, P]),
    "hd_pixel_unshuffle": (None, [P, c_int, c_int, c_int, c_int, P]),
    "hd_decode_to_rgb": (None, [P, c_int, c_int, c_int, c_int, P]),
    "hd_denoise_scratch_bytes": (c_int64, [c_int, c_int, c_int]),
    "hd_denoise_euler_cfg": (c_int, [ctypes.POINTER(hd_forward_binding), ctypes.POINTER(hd_forward_workspace),
                                     P, c_int, P, c_int, P, c_int, P, c_int, c_float, c_int, c_int,
                                     c_int, c_int, c_int, c_int, c_int, P, c_int64, P]),
    "hd_scheduler_unipc_plan": (None, [ctypes.POINTER(hd_scheduler), c_int, c_int, c_int,
                                       ctypes.POINTER(hd_unipc_plan)]),
    "hd_scheduler_unipc_step": (c_int, [ctypes.POINTER(hd_scheduler), ctypes.POINTER(hd_scheduler_unipc),
                                        P, P, P, c_int, P]),
    "hd_step_noise": (None, [ctypes.POINTER(hd_torch_rng), P, c_int64, c_float]),
    "hd_denoise_set_output_check": (c_int, [c_int]),
    "hd_denoise_run_scratch_bytes": (c_int64, [c_int, c_int, c_int, c_int]),
    "hd_denoise": (c_int, [ctypes.POINTER(hd_forward_binding), ctypes.POINTER(hd_forward_workspace), c_int,
                           ctypes.POINTER(hd_scheduler), c_int, c_int, P, c_int, P, c_int, P, c_int,
                           c_float, ctypes.c_uint64, c_float, c_float, c_float, c_int, c_int, c_int,
                           c_int, c_int, c_int, c_int, P, c_int64, P]),
    "hd_denoise_cfg_scratch_bytes": (c_int64, [c_int, c_int, c_int, c_int]),
    "hd_denoise_cfg": (c_int, [ctypes.POINTER(hd_forward_binding), ctypes.POINTER(hd_forward_workspace),
                               ctypes.POINTER(hd_forward_workspace), c_int, ctypes.POINTER(hd_scheduler),
                               c_int, P, c_int, P, c_int, c_int, P, c_int, P, c_int, c_int, P, c_int,
                               c_float, ctypes.c_uint64, c_float, c_float, c_float, c_int, c_int, c_int,
                               c_int, c_int, c_int, P, c_int64, P]),
    "hd_denoise_visual": (c_int, [ctypes.POINTER(hd_forward_binding), ctypes.POINTER(hd_forward_workspace),
                                  c_int, ctypes.POINTER(hd_scheduler), c_int, P, c_int, P, P,
                                  ctypes.POINTER(hd_visual_cond), P, c_int, P, c_int, ctypes.c_uint64,
                                  c_float, c_float, c_float, c_int, c_int, c_int, c_int, c_int, c_int,
                                  c_int, P, c_int64, P]),
    "hd_unipc_convert": (None, [P, P, c_float, P, c_int]),
    "hd_unipc_correct": (None, [P, P, P, P] + [c_float] * 8 + [c_int, P, c_int]),
    # hd_sequence.h
    "hd_resolution_snap": (None, [c_int, c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int)]),
    "hd_seq_t2i": (c_int, [P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                           c_int, ctypes.POINTER(hd_sequence)]),
    "hd_seq_build_tokens": (c_int, [P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                    c_int, c_int, c_int, ctypes.POINTER(hd_ref_geom), ctypes.POINTER(hd_sequence)]),
    "hd_sequence_free": (None, [ctypes.POINTER(hd_sequence)]),
    "hd_seq_diag": (c_int, [ctypes.POINTER(hd_sequence), c_char_p]),
    # hd_vision.h
    "hd_vision_layout": (None, [ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(hd_vision_offsets)]),
    "hd_vision_resolve": (c_int, [ctypes.POINTER(hd_weight_store), ctypes.POINTER(hd_vision_binding)]),
    "hd_vision_workspace_bytes": (ctypes.c_int64, [ctypes.c_int64]),
    "hd_vision_tables_bytes": (ctypes.c_int64, [ctypes.c_int64]),
    "hd_vision_prepare_tables": (c_int, [ctypes.POINTER(hd_vision_workspace), c_int, c_int, c_int]),
    "hd_vision_forward": (c_int, [ctypes.POINTER(hd_vision_binding), ctypes.POINTER(hd_vision_workspace),
                                  P, c_int, c_int, c_int, P, ctypes.POINTER(P)]),
    "hd_vision_forward_multi": (c_int, [ctypes.POINTER(hd_vision_binding), ctypes.POINTER(hd_vision_workspace),
                                        P, c_int, c_int, c_int, c_int, P, ctypes.POINTER(P)]),
    "hd_vision_workspace_bytes_multi": (ctypes.c_int64, [c_int, ctypes.c_int64]),
    "hd_vision_patch": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_vision_layernorm": (None, [P, P, P, P, c_int, c_int, c_float]),
    "hd_vision_gelu": (None, [P, P, c_size_t]),
    "hd_vision_gelu_exact": (None, [P, P, c_size_t]),
    "hd_vision_pos_interp": (None, [P, P, P, P, c_int, c_int]),
    "hd_vision_rot": (None, [P, P, P, c_int, c_int]),
    "hd_vision_rot_cos_sin": (None, [P, P, P, c_int, c_int]),
    "hd_vision_spatial_merge": (None, [P, P, c_int, c_int, c_int]),
    "hd_vision_qkv_split": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_vision_attn_merge": (None, [P, P, c_int, c_int, c_int]),
    "hd_vision_masked_scatter": (None, [P, P, P, P, c_int, c_int]),
    "hd_vision_deepstack_inject": (None, [P, P, P, P, c_int, c_int]),
    "hd_vision_masked_scatter_n": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_vision_deepstack_inject_n": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_linear_ld": (None, [P, P, P, P, c_int, c_int, c_int, c_int]),
    "hd_linear_ws": (None, [P, P, P, P, c_int, c_int, c_int, P, ctypes.c_int64]),
    "hd_linear_residual_ws": (None, [P, P, P, P, c_int, c_int, c_int, P, ctypes.c_int64]),
    "hd_gemm_ws_bytes": (ctypes.c_int64, []),
    "hd_linear_noalloc": (None, [P, P, P, P, c_int, c_int, c_int]),
    "hd_linear_noalloc_scratch_bytes": (ctypes.c_int64, []),
    "hd_unipc_predict": (None, [P, P, P] + [c_float] * 7 + [c_int, P, c_int]),
}

_lib = None


def load(path=None):
    """Loads libo1hip.so once and types every exported entry point.
    Raises RuntimeError when the library (the HIP build) is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(
            f"libo1hip.so not found at {p}: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def bind_torch_stream():
    """Makes every later launch of the library go to torch's current stream
    on the current device, so library kernels order with torch's own work."""
    import torch
    load().hd_hip_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def ptr(t):
    """Device pointer of a torch tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def np_ptr(a):
    """Host pointer of a contiguous numpy array."""
    return ctypes.c_void_p(a.ctypes.data)


def randn(seed, n):
    """torch CPU randn(n) from manual_seed(seed), via the library's host RNG."""
    import numpy as np
    g = hd_torch_rng()
    load().hd_torch_rng_seed(ctypes.byref(g), seed)
    out = np.empty(n, np.float32)
    load().hd_torch_randn_f32(ctypes.byref(g), np_ptr(out), n)
    return out


def check_prim(what=""):
    """Raises if a primitive reported an error through the shared buffer."""
    msg = load().hd_cuda_last_error()
    if msg:
        load().hd_cuda_clear_error()
        raise RuntimeError(f"{what}: {msg.decode()}")


def check_status(st, what=""):
    if st != HD_OK:
        raise RuntimeError(f"{what}: status {st}: {load().hd_last_error().decode()}")


# ---------------------------------------------------------------------------
# thin typed helpers (torch tensors in, torch tensors out)
# ---------------------------------------------------------------------------
def _torch():
    import torch
    return torch


def linear(x, w, bias=None, out=None):
    t = _torch()
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = t.empty((M, N), dtype=t.bfloat16, device=x.device)
    load().hd_linear(ptr(x), ptr(w), ptr(bias), ptr(out), M, N, K, 1)
    check_prim("hd_linear")
    return out


def block_config(eps=1e-6, theta=5e6, attention_scaling=1.0, section=(24, 20, 20), interleaved=1):
    c = hd_block_config()
    c.eps, c.rope_theta, c.attention_scaling = eps, theta, attention_scaling
    for i in range(3):
        c.section[i] = section[i]
    c.interleaved = interleaved
    return c


def set_block_config(**kw):
    c = block_config(**kw)
    load().hd_block_set_config(ctypes.byref(c))
    return c


def binding_from(weights, layer_idx=0):
    """weights: dict of device tensors with the hd_block_binding field names."""
    b = hd_block_binding()
    b.layer_idx = layer_idx
    for n, _ in hd_block_binding._fields_[1:]:
        setattr(b, n, weights[n].data_ptr())
    return b


class WeightStore:
    """hd_weight_store over named torch device tensors (caller keeps them)."""

    def __init__(self, named):
        self.named = dict(named)
        arr = (hd_device_alloc * len(self.named))()
        for i, (n, t) in enumerate(self.named.items()):
            arr[i].dev_ptr = t.data_ptr()
            arr[i].nbytes = t.numel() * t.element_size()
            arr[i].name = n.encode()
        self._arr = arr
        self.store = hd_weight_store()
        self.store.device_id = 0
        self.store.allocs = ctypes.cast(arr, ctypes.POINTER(hd_device_alloc))
        self.store.n_allocs = len(self.named)


def rope_table(pos, seq, head_dim=128, theta=5e6, section=(24, 20, 20), interleaved=1,
               attention_scaling=1.0, out=None):
    t = _torch()
    if out is None:
        out = t.empty((seq, head_dim // 2, 2), dtype=t.float32, device=pos.device)
    sec = (ctypes.c_int64 * 3)(*section)
    load().hd_rope_table(ptr(pos), seq, sec, 3, head_dim, theta, attention_scaling, interleaved,
                         ptr(out))
    check_prim("hd_rope_table")
    return out


class SdpaPlan:
    def __init__(self, batch, q_heads, kv_heads, seq, head_dim=128, scale=None, ar_len=0):
        self.h = c_void_p()
        scale = scale if scale is not None else head_dim ** -0.5
        rc = load().hd_sdpa_create_prod(ctypes.byref(self.h), batch, q_heads, kv_heads, seq,
                                        ar_len, head_dim, scale)
        if rc != 0:
            raise RuntimeError(load().hd_cuda_last_error().decode())

    def __del__(self):
        try:
            if getattr(self, "h", None) and _lib is not None:
                _lib.hd_sdpa_destroy(self.h)
                self.h = None
        except (AttributeError, TypeError):     # interpreter shutdown
            pass

"""ctypes declarations of the C ABI in include/voxhip.h.

Struct layouts and prototypes mirror the header one to one; tests compare the
struct sizes/offsets against a C compiler and the prototypes against the
symbols the shared library exports.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

u32, u64, f32, f64, i32 = C.c_uint32, C.c_uint64, C.c_float, C.c_double, C.c_int
vp = C.c_void_p

LIB_PATH = Path(__file__).resolve().parent / "libvoxhip.so"

VX_OK = 0
STATUS = {
    0: "VX_OK", -1: "VX_ERR_INVALID_ARG", -2: "VX_ERR_HIP", -3: "VX_ERR_OOM", -4: "VX_ERR_SHAPE",
    -5: "VX_ERR_BOUNDS", -6: "VX_ERR_UNSUPPORTED", -7: "VX_ERR_CONTEXT_FULL",
    -8: "VX_ERR_TOKEN_RANGE", -9: "VX_ERR_GGUF", -10: "VX_ERR_NOT_FOUND", -11: "VX_ERR_OFFSET",
    -12: "VX_ERR_CANCELLED", -13: "VX_ERR_NO_DEVICE", -14: "VX_ERR_STATE",
}
STATUS_CODE = {v: k for k, v in STATUS.items()}

DTYPE_F32, DTYPE_F16, DTYPE_Q8_0 = 0, 1, 8
EXEC_GRAPH, EXEC_FUSED, EXEC_REFERENCE, EXEC_PERSISTENT = 0, 1, 2, 3
PREFILL_AUTO, PREFILL_TILES, PREFILL_STREAMK_TAIL_FIRST = 0, 1, 2
BUF = dict(HIDDEN=0, NORM=1, Q=2, K=3, V=4, ATTENTION=5, GATE=6, BRANCH=7, LOGITS=8,
           SCORES=9, KV_K=10, KV_V=11, POSITION=12)


def _struct(name, fields):
    return type(name, (C.Structure,), {"_fields_": fields})


EmbeddingPush = _struct("EmbeddingPush", [("weight_offset", u32), ("cols", u32), ("token_id", u32),
                                          ("dtype", u32), ("alpha", f32)])
RmsPush = _struct("RmsPush", [("weight_offset", u32), ("n", u32), ("eps", f32)])
MatvecPush = _struct("MatvecPush", [("weight_offset", u32), ("rows", u32), ("cols", u32),
                                    ("dtype", u32), ("row_base", u32), ("alpha", f32)])
RopePush = _struct("RopePush", [("factor_offset", u32), ("position", u32), ("q_heads", u32),
                                ("kv_heads", u32), ("head_dim", u32), ("rope_theta", f32),
                                ("scaling_factor", f32)])
StoreKvPush = _struct("StoreKvPush", [("layer", u32), ("position", u32), ("context", u32),
                                      ("kv_dim", u32)])
AttentionPush = _struct("AttentionPush", [("layer", u32), ("context", u32), ("position", u32),
                                          ("head_dim", u32), ("q_per_kv", u32), ("kv_heads", u32)])
SoftmaxPush = _struct("SoftmaxPush", [("context", u32), ("position", u32)])
QkvPush = _struct("QkvPush", [("q_weight_offset", u32), ("k_weight_offset", u32),
                              ("v_weight_offset", u32), ("q_rows", u32), ("kv_rows", u32),
                              ("cols", u32), ("q_dtype", u32), ("k_dtype", u32), ("v_dtype", u32),
                              ("row_base", u32)])
SwigluPush = _struct("SwigluPush", [("gate_weight_offset", u32), ("up_weight_offset", u32),
                                    ("rows", u32), ("cols", u32), ("dtype", u32), ("row_base", u32)])
ResidualRmsPush = _struct("ResidualRmsPush", [("weight_offset", u32), ("n", u32), ("eps", f32),
                                              ("scale", f32)])
LinearBiasPush = _struct("LinearBiasPush", [("weight_offset", u32), ("bias_offset", u32),
                                            ("rows", u32), ("cols", u32), ("weight_dtype", u32),
                                            ("bias_dtype", u32), ("row_base", u32), ("alpha", f32)])
FusionPush = _struct("FusionPush", [("weight_offset", u32), ("bias_offset", u32), ("rows", u32),
                                    ("left_cols", u32), ("right_cols", u32), ("weight_dtype", u32),
                                    ("bias_dtype", u32), ("row_base", u32)])
# Token-batched push structs (local.rs:183-200).
SeqLinearPush = _struct("SeqLinearPush", [(n, u32) for n in (
    "weight_offset", "bias_offset", "rows", "cols", "weight_dtype", "bias_dtype", "tokens",
    "input_stride", "output_stride", "input_base", "output_base", "has_bias")] + [("alpha", f32)])
SeqRmsPush = _struct("SeqRmsPush", [(n, u32) for n in (
    "weight_offset", "n", "tokens", "input_stride", "output_stride", "input_base",
    "output_base")] + [("eps", f32)])
SeqResidualRmsPush = _struct("SeqResidualRmsPush", [(n, u32) for n in (
    "weight_offset", "n", "tokens", "hidden_stride", "branch_stride", "output_stride",
    "hidden_base", "branch_base", "output_base")] + [("eps", f32), ("scale", f32)])
SeqQkvPush = _struct("SeqQkvPush", [(n, u32) for n in (
    "q_weight_offset", "k_weight_offset", "v_weight_offset", "q_rows", "kv_rows", "cols", "tokens",
    "input_stride", "q_stride", "kv_stride", "input_base")])
SeqSwigluPush = _struct("SeqSwigluPush", [(n, u32) for n in (
    "gate_weight_offset", "up_weight_offset", "rows", "cols", "tokens", "input_stride",
    "output_stride", "input_base", "output_base")])
SeqRopePush = _struct("SeqRopePush", [(n, u32) for n in (
    "factor_offset", "tokens", "q_heads", "kv_heads", "head_dim", "q_stride", "k_stride")] +
    [("rope_theta", f32), ("scaling_factor", f32)])
DenseScoresPush = _struct("DenseScoresPush", [(n, u32) for n in (
    "tokens", "q_heads", "kv_heads", "head_dim", "q_stride", "k_stride", "score_stride")])
DenseSoftmaxPush = _struct("DenseSoftmaxPush", [(n, u32) for n in ("tokens", "q_heads", "score_stride")])
DenseValuesPush = _struct("DenseValuesPush", [(n, u32) for n in (
    "tokens", "q_heads", "kv_heads", "head_dim", "out_stride", "v_stride", "score_stride")])
CfmNoisePush = _struct("CfmNoisePush", [("n", u32), ("seed_lo", u32), ("seed_hi", u32), ("temperature", f32)])
CfmEulerPush = _struct("CfmEulerPush", [("n", u32), ("dt", f32), ("cfg", f32), ("use_zero_star", u32)])
TimePush = _struct("TimePush", [("dim", u32), ("t", f32)])
PackLocDitPush = _struct("PackLocDitPush", [("hidden", u32), ("patch_tokens", u32), ("zero_mu", u32)])
LocDitConfig = _struct("LocDitConfig", [(n, u32) for n in (
    "hidden", "layers", "q_heads", "kv_heads", "head_dim", "ffn", "feat_dim", "patch", "n_mu", "n_cond",
    "cond_raw", "uncond_zero_cond")] + [("rms_epsilon", f32), ("rope_theta", f32), ("rope_scaling", f32)])
CfmOptions = _struct("CfmOptions", [("n_timesteps", u32), ("cfg_value", f32), ("temperature", f32),
                                    ("sway_sampling_coef", f32), ("seed", u64), ("use_cfg_zero_star", u32)])
CfmResult = _struct("CfmResult", [("elapsed_ms", f64), ("n_timesteps", u32), ("estimator_calls", u32),
                                  ("zero_init_steps", u32), ("output_checksum", f64), ("output_l2", f64),
                                  ("output_min", f32), ("output_max", f32)])
DeviceInfo = _struct("DeviceInfo", [("name", C.c_char * 256), ("arch", C.c_char * 64),
                                    ("total_global_mem", u64), ("compute_units", u32),
                                    ("wavefront_size", u32), ("l2_cache_bytes", u32),
                                    ("lds_bytes_per_block", u32), ("clock_khz", u32),
                                    ("memory_clock_khz", u32), ("memory_bus_width", u32)])
ProfEntry = _struct("ProfEntry", [("name", C.c_char * 64), ("total_ms", f64), ("calls", u64),
                                  ("avg_ms", f64)])
TensorInfo = _struct("TensorInfo", [("name", C.c_char * 96), ("ggml_type", u32), ("n_dims", u32),
                                    ("dims", u64 * 4), ("offset", u64), ("bytes", u64)])
FusedQkvArgs = _struct("FusedQkvArgs", [("norm_offset", u32), ("eps", f32),
                                        ("q_weight_offset", u32), ("k_weight_offset", u32),
                                        ("v_weight_offset", u32), ("q_rows", u32), ("kv_rows", u32),
                                        ("cols", u32), ("dtype", u32), ("factor_offset", u32),
                                        ("head_dim", u32), ("rope_theta", f32),
                                        ("scaling_factor", f32), ("layer", u32), ("context", u32)])
FusedAttnArgs = _struct("FusedAttnArgs", [("layer", u32), ("context", u32), ("head_dim", u32),
                                          ("q_heads", u32), ("kv_heads", u32), ("splits", u32)])
FusedResidualArgs = _struct("FusedResidualArgs", [("weight_offset", u32), ("rows", u32),
                                                  ("cols", u32), ("dtype", u32), ("scale", f32)])
FusedSwigluArgs = _struct("FusedSwigluArgs", [("norm_offset", u32), ("eps", f32),
                                              ("gate_weight_offset", u32),
                                              ("up_weight_offset", u32), ("rows", u32),
                                              ("cols", u32), ("dtype", u32)])
GgufSummary = _struct("GgufSummary", [("version", u32), ("tensor_count", u64),
                                      ("metadata_count", u64), ("alignment", u64),
                                      ("data_offset", u64), ("file_bytes", u64),
                                      ("tensor_bytes", u64)])
BaseLmConfig = _struct("BaseLmConfig", [
    ("context_length", u32), ("active_context_length", u32), ("embedding_length", u32),
    ("block_count", u32), ("feed_forward_length", u32), ("vocab_size", u32), ("head_count", u32),
    ("head_count_kv", u32), ("head_dim", u32), ("kv_dim", u32), ("rms_epsilon", f32),
    ("rope_theta", f32), ("rope_dimension_count", u32), ("rope_original_context_length", u32),
    ("rope_longrope", u32), ("embedding_scale", f32), ("residual_scale", f32),
    ("logit_scale", f32), ("tied_output", u32)])
BaseLmOptions = _struct("BaseLmOptions", [("exec_mode", u32), ("strict_geometry", u32),
                                          ("attn_splits", u32), ("prefill_schedule", u32)])
TopLogit = _struct("TopLogit", [("token_id", u32), ("logit", f32)])
StepResult = _struct("StepResult", [("position", u32), ("elapsed_ms", f64),
                                    ("final_hidden_checksum", f64), ("final_hidden_l2", f64),
                                    ("n_top", u32)])
BenchmarkResult = _struct("BenchmarkResult", [("iterations", u32), ("token_id", u32),
                                              ("mean_ms", f64), ("min_ms", f64), ("max_ms", f64),
                                              ("tokens_per_second", f64)])
FsqPush = _struct("FsqPush", [("n", u32), ("scale", f32)])
AcousticConfig = _struct("AcousticConfig", [
    ("model_version", f32), ("residual_block_count", u32), ("embedding_length", u32),
    ("feed_forward_length", u32), ("head_count", u32), ("head_count_kv", u32), ("head_dim", u32),
    ("kv_dim", u32), ("no_rope", u32), ("active_context_length", u32), ("rms_epsilon", f32),
    ("residual_scale", f32), ("fsq_latent_dim", u32), ("fsq_scale", f32), ("fusion_input_dim", u32)])
ResidualOptions = _struct("ResidualOptions", [("exec_mode", u32), ("strict_geometry", u32)])
FsqResult = _struct("FsqResult", [("elapsed_ms", f64), ("output_checksum", f64), ("output_l2", f64),
                                  ("latent_checksum", f64), ("latent_l2", f64)])
ResidualStepResult = _struct("ResidualStepResult", [
    ("position", u32), ("fsq_applied", u32), ("elapsed_ms", f64), ("fsq_checksum", f64), ("fsq_l2", f64),
    ("fused_input_checksum", f64), ("fused_input_l2", f64), ("residual_hidden_checksum", f64),
    ("residual_hidden_l2", f64)])
ResidualGpuStep = _struct("ResidualGpuStep", [("position", u32), ("fsq_applied", u32), ("elapsed_ms", f64)])
ResidualBenchmark = _struct("ResidualBenchmark", [("iterations", u32), ("mean_ms", f64), ("min_ms", f64),
                                                  ("max_ms", f64), ("steps_per_second", f64)])
StopPrediction = _struct("StopPrediction", [("stop", u32), ("continue_logit", f32), ("stop_logit", f32),
                                            ("elapsed_ms", f64)])
VaeConvPush = _struct("VaeConvPush", [(n, u32) for n in (
    "weight_offset", "bias_offset", "in_channels", "out_channels", "in_length", "out_length", "kernel", "stride",
    "dilation", "groups", "left_pad", "weight_dtype", "bias_dtype", "has_bias")])
VaeConvTPush = _struct("VaeConvTPush", [(n, u32) for n in (
    "weight_offset", "bias_offset", "in_channels", "out_channels", "in_length", "out_length", "kernel", "stride",
    "groups", "weight_dtype", "bias_dtype", "has_bias")])
VaeSnakePush = _struct("VaeSnakePush", [(n, u32) for n in ("alpha_offset", "channels", "length", "dtype")])
VaeScalePush = _struct("VaeScalePush", [(n, u32) for n in (
    "scale_offset", "bias_offset", "channels", "length", "bucket", "buckets", "scale_dtype", "bias_dtype")])
VaeGridPush = _struct("VaeGridPush", [("channels", u32), ("length", u32)])
AudioVaeConfig = _struct("AudioVaeConfig", [
    ("encoder_dim", u32), ("latent_dim", u32), ("decoder_dim", u32), ("sample_rate", u32),
    ("out_sample_rate", u32), ("encoder_rates", u32 * 4), ("decoder_rates", u32 * 6), ("encoder_hop", u32),
    ("decoder_hop", u32), ("patch_size", u32), ("input_samples_per_patch", u32),
    ("output_samples_per_patch", u32), ("sr_bin_boundaries", u32 * 3), ("decoder_sr_bucket", u32),
    ("depthwise", u32)])
AudioDecodeStats = _struct("AudioDecodeStats", [
    ("latent_frames", u32), ("latent_patches", u32), ("output_samples", u32), ("output_sample_rate", u32),
    ("duration_seconds", f64), ("checksum", f64), ("l2", f64), ("peak", f32), ("decode_ms", f64),
    ("scratch_bytes", u64)])
RESIDUAL_BUF = dict(OUTPUT=0, CURRENT_LM=1, FSQ_LATENT=2, FSQ_OUTPUT=3, FUSION_SNAPSHOT=4, HIDDEN=5,
                    KV_K=6, KV_V=7, STOP_LOGITS=8)

P = C.POINTER
CTX = vp   # vx_ctx*
BUFP = vp  # vx_buf*
MODEL = vp
GRAPH = vp
ENGINE = vp
GGUF = vp
LOCDIT = vp
RESIDUAL = vp
AUDIOVAE = vp

# name -> (restype, argtypes)
PROTOTYPES = {
    "vx_abi_version": (i32, []),
    "vx_last_error": (C.c_char_p, []),
    "vx_init": (i32, [i32, P(CTX)]),
    "vx_destroy": (i32, [CTX]),
    "vx_device_info_get": (i32, [CTX, P(DeviceInfo)]),
    "vx_alloc": (i32, [CTX, u64, P(BUFP)]),
    "vx_free": (i32, [CTX, BUFP]),
    "vx_buf_size": (u64, [BUFP]),
    "vx_buf_device_ptr": (vp, [BUFP]),
    "vx_upload": (i32, [CTX, BUFP, u64, vp, u64]),
    "vx_download": (i32, [CTX, BUFP, u64, vp, u64]),
    "vx_copy": (i32, [CTX, BUFP, u64, BUFP, u64, u64]),
    "vx_fill_u32": (i32, [CTX, BUFP, u64, u32, u64]),
    "vx_sync": (i32, [CTX]),
    "vx_set_cancel_flag": (i32, [CTX, P(u32)]),
    "vx_graph_begin": (i32, [CTX]),
    "vx_graph_end": (i32, [CTX, P(GRAPH)]),
    "vx_graph_launch": (i32, [CTX, GRAPH]),
    "vx_graph_free": (i32, [CTX, GRAPH]),
    "vx_prof_enable": (i32, [CTX, i32]),
    "vx_prof_reset": (i32, [CTX]),
    "vx_prof_snapshot": (i32, [CTX, P(ProfEntry), u32, P(u32)]),
    "vx_model_upload": (i32, [CTX, vp, u64, P(TensorInfo), u32, P(MODEL)]),
    "vx_model_free": (i32, [CTX, MODEL]),
    "vx_model_tensor_count": (u32, [MODEL]),
    "vx_model_tensor_at": (i32, [MODEL, u32, P(TensorInfo)]),
    "vx_model_find": (i32, [MODEL, C.c_char_p, P(TensorInfo)]),
    "vx_model_device_bytes": (u64, [MODEL]),
    "vx_dequant": (i32, [CTX, MODEL, u32, u32, u32, u32, BUFP]),
    "vx_embedding": (i32, [CTX, MODEL, BUFP, P(EmbeddingPush)]),
    "vx_embedding_devtok": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, P(EmbeddingPush)]),
    "vx_rmsnorm": (i32, [CTX, MODEL, BUFP, BUFP, P(RmsPush)]),
    "vx_residual_rmsnorm": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, P(ResidualRmsPush)]),
    "vx_matvec": (i32, [CTX, MODEL, BUFP, BUFP, P(MatvecPush)]),
    "vx_qkv_matvec": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, BUFP, P(QkvPush)]),
    "vx_matvec_swiglu": (i32, [CTX, MODEL, BUFP, BUFP, P(SwigluPush)]),
    "vx_rope": (i32, [CTX, MODEL, BUFP, BUFP, P(RopePush)]),
    "vx_rope_devpos": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, P(RopePush)]),
    "vx_store_kv": (i32, [CTX, BUFP, BUFP, BUFP, BUFP, P(StoreKvPush)]),
    "vx_store_kv_devpos": (i32, [CTX, BUFP, BUFP, BUFP, BUFP, BUFP, P(StoreKvPush)]),
    "vx_attn_scores": (i32, [CTX, BUFP, BUFP, BUFP, P(AttentionPush)]),
    "vx_attn_scores_devpos": (i32, [CTX, BUFP, BUFP, BUFP, BUFP, P(AttentionPush)]),
    "vx_softmax": (i32, [CTX, BUFP, u32, P(SoftmaxPush)]),
    "vx_softmax_devpos": (i32, [CTX, BUFP, u32, BUFP, P(SoftmaxPush)]),
    "vx_attn_values": (i32, [CTX, BUFP, BUFP, BUFP, P(AttentionPush)]),
    "vx_attn_values_devpos": (i32, [CTX, BUFP, BUFP, BUFP, BUFP, P(AttentionPush)]),
    "vx_linear_bias": (i32, [CTX, MODEL, BUFP, BUFP, P(LinearBiasPush)]),
    "vx_fusion_linear": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, BUFP, P(FusionPush)]),
    "vx_seq_linear_bias": (i32, [CTX, MODEL, BUFP, BUFP, P(SeqLinearPush)]),
    "vx_seq_qkv": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, BUFP, P(SeqQkvPush)]),
    "vx_seq_swiglu": (i32, [CTX, MODEL, BUFP, BUFP, P(SeqSwigluPush)]),
    "vx_seq_silu_mul": (i32, [CTX, BUFP, BUFP, u32]),
    "vx_seq_rmsnorm": (i32, [CTX, MODEL, BUFP, BUFP, P(SeqRmsPush)]),
    "vx_seq_residual_rmsnorm": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, P(SeqResidualRmsPush)]),
    "vx_seq_rope": (i32, [CTX, MODEL, BUFP, BUFP, P(SeqRopePush)]),
    "vx_seq_rope_at": (i32, [CTX, MODEL, BUFP, BUFP, u32, P(SeqRopePush)]),
    "vx_dense_attn_scores": (i32, [CTX, BUFP, BUFP, BUFP, P(DenseScoresPush)]),
    "vx_dense_softmax": (i32, [CTX, BUFP, P(DenseSoftmaxPush)]),
    "vx_dense_attn_values": (i32, [CTX, BUFP, BUFP, BUFP, P(DenseValuesPush)]),
    "vx_cfm_noise": (i32, [CTX, BUFP, P(CfmNoisePush)]),
    "vx_cfm_cfg_euler": (i32, [CTX, BUFP, BUFP, BUFP, P(CfmEulerPush)]),
    "vx_time_sinusoidal": (i32, [CTX, BUFP, P(TimePush)]),
    "vx_pack_locdit": (i32, [CTX, BUFP, BUFP, BUFP, BUFP, BUFP, BUFP, P(PackLocDitPush)]),
    "vx_silu_inplace": (i32, [CTX, BUFP, u32]),
    "vx_add_vectors": (i32, [CTX, BUFP, BUFP, u32]),
    "vx_locdit_create": (i32, [CTX, MODEL, MODEL, u32, P(LocDitConfig), u32, P(LOCDIT)]),
    "vx_locdit_destroy": (i32, [LOCDIT]),
    "vx_locdit_estimate": (i32, [LOCDIT, P(f32), P(f32), P(f32), f32, f32, P(f32)]),
    "vx_locdit_cfm_solve": (i32, [LOCDIT, P(f32), P(f32), P(CfmOptions), P(f32), P(f32), P(CfmResult)]),
    "vx_locdit_cfm_solve_from_model_hiddens": (i32, [LOCDIT, BUFP, BUFP, P(f32), P(CfmOptions), P(f32), P(f32),
                                                     P(CfmResult)]),
    "vx_fused_qkv_rope_store": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, BUFP, BUFP, BUFP, BUFP,
                                      P(FusedQkvArgs)]),
    "vx_fused_attention_scratch_bytes": (u64, [P(FusedAttnArgs)]),
    "vx_fused_attention": (i32, [CTX, BUFP, BUFP, BUFP, BUFP, BUFP, BUFP, P(FusedAttnArgs)]),
    "vx_fused_attention_noalloc": (i32, [CTX, BUFP, BUFP, BUFP, BUFP, BUFP, P(FusedAttnArgs)]),
    "vx_fused_matvec_residual": (i32, [CTX, MODEL, BUFP, BUFP, BUFP, P(FusedResidualArgs)]),
    "vx_fused_rms_swiglu": (i32, [CTX, MODEL, BUFP, BUFP, P(FusedSwigluArgs)]),
    "vx_diag_stream_read": (i32, [CTX, BUFP, u64, u64, BUFP, u32, u32]),
    "vx_diag_stream_copy": (i32, [CTX, BUFP, BUFP, u64, u32]),
    "vx_diag_timeline_arm": (i32, [CTX, u64]),
    "vx_diag_timeline_read": (i32, [CTX, P(u64), u64, P(u64), u64, P(u64), P(u64)]),
    "vx_gguf_open": (i32, [C.c_char_p, P(GGUF)]),
    "vx_gguf_close": (i32, [GGUF]),
    "vx_gguf_summary_get": (i32, [GGUF, P(GgufSummary)]),
    "vx_gguf_tensor_at": (i32, [GGUF, u32, P(TensorInfo)]),
    "vx_gguf_find": (i32, [GGUF, C.c_char_p, P(TensorInfo)]),
    "vx_gguf_meta": (i32, [GGUF, C.c_char_p, C.c_char_p, u32]),
    "vx_gguf_primary_format": (i32, [GGUF, P(u32)]),
    "vx_model_upload_gguf": (i32, [CTX, GGUF, P(MODEL)]),
    "vx_baselm_config_from_gguf": (i32, [GGUF, u32, P(BaseLmConfig)]),
    "vx_baselm_rope_scaling_factor": (f32, [P(BaseLmConfig)]),
    "vx_baselm_kv_cache_bytes": (u64, [P(BaseLmConfig)]),
    "vx_top_k_logits": (i32, [P(f32), u32, u32, P(TopLogit), P(u32)]),
    "vx_baselm_create": (i32, [CTX, MODEL, P(BaseLmConfig), P(BaseLmOptions), P(ENGINE)]),
    "vx_baselm_destroy": (i32, [ENGINE]),
    "vx_baselm_reset": (i32, [ENGINE]),
    "vx_baselm_position": (u32, [ENGINE]),
    "vx_baselm_set_position": (i32, [ENGINE, u32]),
    "vx_baselm_decode_token": (i32, [ENGINE, u32, u32, P(StepResult), P(TopLogit)]),
    "vx_baselm_decode_embedding": (i32, [ENGINE, P(f32), u32, u32, P(StepResult), P(TopLogit)]),
    "vx_baselm_decode_token_gpu_only": (i32, [ENGINE, u32, P(u32)]),
    "vx_baselm_decode_embedding_gpu_only": (i32, [ENGINE, P(f32), u32, P(u32)]),
    "vx_baselm_decode_embedding_from_gpu_only": (i32, [ENGINE, BUFP, P(u32)]),
    "vx_baselm_decode_tokens_gpu_only": (i32, [ENGINE, P(u32), u32]),
    "vx_baselm_prefill_tokens": (i32, [ENGINE, P(u32), u32, u32, P(StepResult), P(TopLogit)]),
    "vx_baselm_prefill_tokens_batched": (i32, [ENGINE, P(u32), u32, u32, P(StepResult), P(TopLogit)]),
    "vx_baselm_prefill_tokens_batched_gpu_only": (i32, [ENGINE, P(u32), u32]),
    "vx_baselm_benchmark": (i32, [ENGINE, u32, u32, u32, P(BenchmarkResult)]),
    "vx_baselm_buffer": (BUFP, [ENGINE, u32]),
    "vx_baselm_profile_steps": (i32, [ENGINE, P(u32), u32, P(ProfEntry), u32, P(u32)]),
    "vx_baselm_time_layer_kernel": (i32, [ENGINE, u32, u32, P(C.c_double)]),
    "vx_fsq_quantize": (i32, [CTX, BUFP, P(FsqPush)]),
    "vx_acoustic_config_from_gguf": (i32, [GGUF, P(BaseLmConfig), u32, P(AcousticConfig)]),
    "vx_acoustic_kv_cache_bytes": (u64, [P(AcousticConfig)]),
    "vx_residual_create": (i32, [CTX, MODEL, P(AcousticConfig), P(ResidualOptions), P(RESIDUAL)]),
    "vx_residual_destroy": (i32, [RESIDUAL]),
    "vx_residual_position": (u32, [RESIDUAL]),
    "vx_residual_reset": (i32, [RESIDUAL]),
    "vx_residual_allocated_bytes": (u64, [RESIDUAL]),
    "vx_residual_buffer": (BUFP, [RESIDUAL, u32]),
    "vx_residual_fsq_only": (i32, [RESIDUAL, P(f32), u32, P(FsqResult)]),
    "vx_residual_step": (i32, [RESIDUAL, P(f32), P(f32), u32, P(ResidualStepResult)]),
    "vx_residual_step_from_gpu_base": (i32, [RESIDUAL, BUFP, P(f32), u32, P(ResidualStepResult)]),
    "vx_residual_step_from_gpu_base_and_embedding": (i32, [RESIDUAL, BUFP, BUFP, P(ResidualStepResult)]),
    "vx_residual_step_from_gpu_base_and_embedding_gpu_only": (i32, [RESIDUAL, BUFP, BUFP, P(ResidualGpuStep)]),
    "vx_residual_step_text_prefix_from_gpu_base": (i32, [RESIDUAL, BUFP, P(ResidualStepResult)]),
    "vx_residual_step_text_prefix_from_gpu_base_gpu_only": (i32, [RESIDUAL, BUFP, P(ResidualGpuStep)]),
    "vx_residual_benchmark": (i32, [RESIDUAL, P(f32), P(f32), u32, u32, u32, P(ResidualBenchmark)]),
    "vx_residual_predict_stop_from_gpu_base": (i32, [RESIDUAL, BUFP, P(StopPrediction)]),
    "vx_residual_predict_stop_from_current_lm": (i32, [RESIDUAL, P(StopPrediction)]),
    "vx_residual_prefill_text_from_gpu_rows": (i32, [RESIDUAL, BUFP, u32]),
    "vx_prefill_text_cross_engine": (i32, [ENGINE, RESIDUAL, P(u32), u32]),
    "vx_vae_conv1d": (i32, [CTX, MODEL, BUFP, BUFP, P(VaeConvPush)]),
    "vx_vae_convtranspose1d": (i32, [CTX, MODEL, BUFP, BUFP, P(VaeConvTPush)]),
    "vx_vae_snake": (i32, [CTX, MODEL, BUFP, BUFP, P(VaeSnakePush)]),
    "vx_vae_scale_bias": (i32, [CTX, MODEL, BUFP, P(VaeScalePush)]),
    "vx_vae_add": (i32, [CTX, BUFP, BUFP, P(VaeGridPush)]),
    "vx_vae_tanh": (i32, [CTX, BUFP, u32]),
    "vx_audiovae_config_from_gguf": (i32, [GGUF, P(AudioVaeConfig)]),
    "vx_audiovae_create": (i32, [CTX, MODEL, P(AudioVaeConfig), u32, P(AUDIOVAE)]),
    "vx_audiovae_destroy": (i32, [AUDIOVAE]),
    "vx_audiovae_scratch_bytes": (u64, [AUDIOVAE]),
    "vx_audiovae_decode_latents": (i32, [AUDIOVAE, P(f32), u64, P(f32), u64, P(AudioDecodeStats)]),
    "vx_audiovae_decode_latents_gpu": (i32, [AUDIOVAE, BUFP, u32, BUFP]),
}

STRUCT_SIZES = {  # C name -> ctypes struct
    "vx_embedding_push": EmbeddingPush, "vx_rms_push": RmsPush, "vx_matvec_push": MatvecPush,
    "vx_rope_push": RopePush, "vx_store_kv_push": StoreKvPush,
    "vx_attention_push": AttentionPush, "vx_softmax_push": SoftmaxPush, "vx_qkv_push": QkvPush,
    "vx_swiglu_push": SwigluPush, "vx_residual_rms_push": ResidualRmsPush,
    "vx_linear_bias_push": LinearBiasPush, "vx_fusion_push": FusionPush,
    "vx_seq_linear_push": SeqLinearPush, "vx_seq_rms_push": SeqRmsPush,
    "vx_seq_residual_rms_push": SeqResidualRmsPush, "vx_seq_qkv_push": SeqQkvPush,
    "vx_seq_swiglu_push": SeqSwigluPush, "vx_seq_rope_push": SeqRopePush,
    "vx_dense_scores_push": DenseScoresPush, "vx_dense_softmax_push": DenseSoftmaxPush,
    "vx_dense_values_push": DenseValuesPush, "vx_cfm_noise_push": CfmNoisePush,
    "vx_cfm_euler_push": CfmEulerPush, "vx_time_push": TimePush, "vx_pack_locdit_push": PackLocDitPush,
    "vx_locdit_config": LocDitConfig, "vx_cfm_options": CfmOptions, "vx_cfm_result": CfmResult,
    "vx_device_info": DeviceInfo, "vx_prof_entry": ProfEntry, "vx_tensor_info": TensorInfo,
    "vx_fused_qkv_args": FusedQkvArgs, "vx_fused_attn_args": FusedAttnArgs,
    "vx_fused_residual_args": FusedResidualArgs, "vx_fused_swiglu_args": FusedSwigluArgs,
    "vx_gguf_summary": GgufSummary, "vx_baselm_config": BaseLmConfig,
    "vx_baselm_options": BaseLmOptions, "vx_top_logit": TopLogit, "vx_step_result": StepResult,
    "vx_baselm_benchmark_result": BenchmarkResult, "vx_fsq_push": FsqPush,
    "vx_acoustic_config": AcousticConfig, "vx_residual_options": ResidualOptions,
    "vx_fsq_result": FsqResult, "vx_residual_step_result": ResidualStepResult,
    "vx_residual_gpu_step": ResidualGpuStep, "vx_residual_benchmark_result": ResidualBenchmark,
    "vx_stop_prediction": StopPrediction, "vx_vae_conv_push": VaeConvPush, "vx_vae_convt_push": VaeConvTPush,
    "vx_vae_snake_push": VaeSnakePush, "vx_vae_scale_push": VaeScalePush, "vx_vae_grid_push": VaeGridPush,
    "vx_audiovae_config": AudioVaeConfig, "vx_audio_decode_stats": AudioDecodeStats,
}


class VxError(RuntimeError):
    """A failed C-ABI call: .status is the vx_status code, .name its symbol."""

    def __init__(self, status: int, message: str, func: str):
        self.status = status
        self.name = STATUS.get(status, str(status))
        super().__init__(f"{func}: {self.name}: {message}")


NOALLOC_SCRATCH_BYTES = 2 * 1024 * 1024  # VX_NOALLOC_SCRATCH_BYTES

_LIB = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libvoxhip.so (once). Raises if the library has not been built.

    VOXHIP_LIBRARY, when set, names another build of the same library to load
    (the sanitizer build the CPU tests run under)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = Path(path) if path else Path(os.environ.get("VOXHIP_LIBRARY") or LIB_PATH)
    if not p.exists():
        raise ImportError(f"{p} is missing: build it with `python voxgen_amd/build.py` "
                          "(or __graft_entry__.build()) before using voxgen_amd")
    lib = C.CDLL(str(p))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(status: int, func: str) -> None:
    if status != VX_OK:
        msg = load().vx_last_error()
        raise VxError(status, msg.decode(errors="replace") if msg else "", func)


def call(name: str, *args):
    """Call a status-returning ABI function and raise VxError on failure."""
    st = getattr(load(), name)(*args)
    check(st, name)
    return st

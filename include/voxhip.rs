// voxhip.rs: Rust declarations of the C ABI in voxhip.h (libvoxhip.so).
//
// The drop-in for VoxGen's Vulkan layer (src/vulkan.rs) on the BaseLM compute
// path: src/hip.rs of the reference crate can be this file. Every function and
// struct of voxhip.h appears here in the header's order, with the same parameter
// types and #[repr(C)] field layout. Generated from the header by
// `python tests/test_rust_binding.py --write`; do not edit by hand. Status codes
// are c_int (VX_OK = 0, negative = error; the message is vx_last_error()). Link
// with build.rs:
//     println!("cargo:rustc-link-lib=dylib=voxhip");
//     println!("cargo:rustc-link-search=native=<dir of libvoxhip.so>");
#![allow(non_camel_case_types, non_upper_case_globals, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

// Status codes (vx_status).
pub type VxStatus = c_int;
pub const VX_OK: c_int = 0;
pub const VX_ERR_INVALID_ARG: c_int = -1;
pub const VX_ERR_HIP: c_int = -2;
pub const VX_ERR_OOM: c_int = -3;
pub const VX_ERR_SHAPE: c_int = -4;
pub const VX_ERR_BOUNDS: c_int = -5;
pub const VX_ERR_UNSUPPORTED: c_int = -6;
pub const VX_ERR_CONTEXT_FULL: c_int = -7;
pub const VX_ERR_TOKEN_RANGE: c_int = -8;
pub const VX_ERR_GGUF: c_int = -9;
pub const VX_ERR_NOT_FOUND: c_int = -10;
pub const VX_ERR_OFFSET: c_int = -11;
pub const VX_ERR_CANCELLED: c_int = -12;
pub const VX_ERR_NO_DEVICE: c_int = -13;
pub const VX_ERR_STATE: c_int = -14;

// Constants (#define).
pub const VX_ABI_VERSION: u32 = 2;
pub const VX_DTYPE_F32: u32 = 0;
pub const VX_DTYPE_F16: u32 = 1;
pub const VX_DTYPE_Q8_0: u32 = 8;
pub const VX_NOALLOC_SCRATCH_BYTES: u32 = 2097152;
pub const VX_EXEC_GRAPH: u32 = 0;
pub const VX_EXEC_FUSED: u32 = 1;
pub const VX_EXEC_REFERENCE: u32 = 2;
pub const VX_EXEC_PERSISTENT: u32 = 3;
pub const VX_PREFILL_AUTO: u32 = 0;
pub const VX_PREFILL_TILES: u32 = 1;
pub const VX_PREFILL_STREAMK_TAIL_FIRST: u32 = 2;
pub const VX_BASELM_BUF_HIDDEN: u32 = 0;
pub const VX_BASELM_BUF_NORM: u32 = 1;
pub const VX_BASELM_BUF_Q: u32 = 2;
pub const VX_BASELM_BUF_K: u32 = 3;
pub const VX_BASELM_BUF_V: u32 = 4;
pub const VX_BASELM_BUF_ATTENTION: u32 = 5;
pub const VX_BASELM_BUF_GATE: u32 = 6;
pub const VX_BASELM_BUF_BRANCH: u32 = 7;
pub const VX_BASELM_BUF_LOGITS: u32 = 8;
pub const VX_BASELM_BUF_SCORES: u32 = 9;
pub const VX_BASELM_BUF_KV_K: u32 = 10;
pub const VX_BASELM_BUF_KV_V: u32 = 11;
pub const VX_BASELM_BUF_POSITION: u32 = 12;
pub const VX_LAYER_KERNEL_QKV: u32 = 0;
pub const VX_LAYER_KERNEL_ATTENTION: u32 = 1;
pub const VX_LAYER_KERNEL_ATTN_OUT: u32 = 2;
pub const VX_LAYER_KERNEL_SWIGLU: u32 = 3;
pub const VX_LAYER_KERNEL_DOWN: u32 = 4;
pub const VX_RESIDUAL_BUF_OUTPUT: u32 = 0;
pub const VX_RESIDUAL_BUF_CURRENT_LM: u32 = 1;
pub const VX_RESIDUAL_BUF_FSQ_LATENT: u32 = 2;
pub const VX_RESIDUAL_BUF_FSQ_OUTPUT: u32 = 3;
pub const VX_RESIDUAL_BUF_FUSION_SNAPSHOT: u32 = 4;
pub const VX_RESIDUAL_BUF_HIDDEN: u32 = 5;
pub const VX_RESIDUAL_BUF_KV_K: u32 = 6;
pub const VX_RESIDUAL_BUF_KV_V: u32 = 7;
pub const VX_RESIDUAL_BUF_STOP_LOGITS: u32 = 8;

// Opaque handles.
#[repr(C)] pub struct VxCtx { _p: [u8; 0] }
#[repr(C)] pub struct VxBuf { _p: [u8; 0] }
#[repr(C)] pub struct VxModel { _p: [u8; 0] }
#[repr(C)] pub struct VxGraph { _p: [u8; 0] }
#[repr(C)] pub struct VxBaselm { _p: [u8; 0] }
#[repr(C)] pub struct VxGguf { _p: [u8; 0] }
#[repr(C)] pub struct VxLocdit { _p: [u8; 0] }
#[repr(C)] pub struct VxResidual { _p: [u8; 0] }
#[repr(C)] pub struct VxAudiovae { _p: [u8; 0] }

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxEmbeddingPush {
    pub weight_offset: u32,
    pub cols: u32,
    pub token_id: u32,
    pub dtype: u32,
    pub alpha: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxRmsPush {
    pub weight_offset: u32,
    pub n: u32,
    pub eps: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxMatvecPush {
    pub weight_offset: u32,
    pub rows: u32,
    pub cols: u32,
    pub dtype: u32,
    pub row_base: u32,
    pub alpha: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxRopePush {
    pub factor_offset: u32,
    pub position: u32,
    pub q_heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub rope_theta: f32,
    pub scaling_factor: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxStoreKvPush {
    pub layer: u32,
    pub position: u32,
    pub context: u32,
    pub kv_dim: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxAttentionPush {
    pub layer: u32,
    pub context: u32,
    pub position: u32,
    pub head_dim: u32,
    pub q_per_kv: u32,
    pub kv_heads: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxSoftmaxPush {
    pub context: u32,
    pub position: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxQkvPush {
    pub q_weight_offset: u32,
    pub k_weight_offset: u32,
    pub v_weight_offset: u32,
    pub q_rows: u32,
    pub kv_rows: u32,
    pub cols: u32,
    pub q_dtype: u32,
    pub k_dtype: u32,
    pub v_dtype: u32,
    pub row_base: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxSwigluPush {
    pub gate_weight_offset: u32,
    pub up_weight_offset: u32,
    pub rows: u32,
    pub cols: u32,
    pub dtype: u32,
    pub row_base: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxResidualRmsPush {
    pub weight_offset: u32,
    pub n: u32,
    pub eps: f32,
    pub scale: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxLinearBiasPush {
    pub weight_offset: u32,
    pub bias_offset: u32,
    pub rows: u32,
    pub cols: u32,
    pub weight_dtype: u32,
    pub bias_dtype: u32,
    pub row_base: u32,
    pub alpha: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxFusionPush {
    pub weight_offset: u32,
    pub bias_offset: u32,
    pub rows: u32,
    pub left_cols: u32,
    pub right_cols: u32,
    pub weight_dtype: u32,
    pub bias_dtype: u32,
    pub row_base: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxSeqLinearPush {
    pub weight_offset: u32,
    pub bias_offset: u32,
    pub rows: u32,
    pub cols: u32,
    pub weight_dtype: u32,
    pub bias_dtype: u32,
    pub tokens: u32,
    pub input_stride: u32,
    pub output_stride: u32,
    pub input_base: u32,
    pub output_base: u32,
    pub has_bias: u32,
    pub alpha: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxSeqRmsPush {
    pub weight_offset: u32,
    pub n: u32,
    pub tokens: u32,
    pub input_stride: u32,
    pub output_stride: u32,
    pub input_base: u32,
    pub output_base: u32,
    pub eps: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxSeqResidualRmsPush {
    pub weight_offset: u32,
    pub n: u32,
    pub tokens: u32,
    pub hidden_stride: u32,
    pub branch_stride: u32,
    pub output_stride: u32,
    pub hidden_base: u32,
    pub branch_base: u32,
    pub output_base: u32,
    pub eps: f32,
    pub scale: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxSeqQkvPush {
    pub q_weight_offset: u32,
    pub k_weight_offset: u32,
    pub v_weight_offset: u32,
    pub q_rows: u32,
    pub kv_rows: u32,
    pub cols: u32,
    pub tokens: u32,
    pub input_stride: u32,
    pub q_stride: u32,
    pub kv_stride: u32,
    pub input_base: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxSeqSwigluPush {
    pub gate_weight_offset: u32,
    pub up_weight_offset: u32,
    pub rows: u32,
    pub cols: u32,
    pub tokens: u32,
    pub input_stride: u32,
    pub output_stride: u32,
    pub input_base: u32,
    pub output_base: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxSeqRopePush {
    pub factor_offset: u32,
    pub tokens: u32,
    pub q_heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub q_stride: u32,
    pub k_stride: u32,
    pub rope_theta: f32,
    pub scaling_factor: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxDenseScoresPush {
    pub tokens: u32,
    pub q_heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub q_stride: u32,
    pub k_stride: u32,
    pub score_stride: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxDenseSoftmaxPush {
    pub tokens: u32,
    pub q_heads: u32,
    pub score_stride: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxDenseValuesPush {
    pub tokens: u32,
    pub q_heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub out_stride: u32,
    pub v_stride: u32,
    pub score_stride: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxCfmNoisePush {
    pub n: u32,
    pub seed_lo: u32,
    pub seed_hi: u32,
    pub temperature: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxCfmEulerPush {
    pub n: u32,
    pub dt: f32,
    pub cfg: f32,
    pub use_zero_star: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxTimePush {
    pub dim: u32,
    pub t: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxPackLocditPush {
    pub hidden: u32,
    pub patch_tokens: u32,
    pub zero_mu: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_abi_version() -> c_int;
    pub fn vx_last_error() -> *const c_char;
    pub fn vx_init(device_index: c_int, out: *mut *mut VxCtx) -> c_int;
    pub fn vx_destroy(ctx: *mut VxCtx) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxDeviceInfo {
    pub name: [c_char; 256],
    pub arch: [c_char; 64],
    pub total_global_mem: u64,
    pub compute_units: u32,
    pub wavefront_size: u32,
    pub l2_cache_bytes: u32,
    pub lds_bytes_per_block: u32,
    pub clock_khz: u32,
    pub memory_clock_khz: u32,
    pub memory_bus_width: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_device_info_get(ctx: *mut VxCtx, out: *mut VxDeviceInfo) -> c_int;
    pub fn vx_alloc(ctx: *mut VxCtx, bytes: u64, out: *mut *mut VxBuf) -> c_int;
    pub fn vx_free(ctx: *mut VxCtx, buf: *mut VxBuf) -> c_int;
    pub fn vx_buf_size(buf: *const VxBuf) -> u64;
    pub fn vx_buf_device_ptr(buf: *const VxBuf) -> *mut c_void;
    pub fn vx_upload(
        ctx: *mut VxCtx,
        dst: *mut VxBuf,
        dst_offset: u64,
        src: *const c_void,
        bytes: u64,
    ) -> c_int;
    pub fn vx_download(
        ctx: *mut VxCtx,
        src: *const VxBuf,
        src_offset: u64,
        dst: *mut c_void,
        bytes: u64,
    ) -> c_int;
    pub fn vx_copy(
        ctx: *mut VxCtx,
        dst: *mut VxBuf,
        dst_offset: u64,
        src: *const VxBuf,
        src_offset: u64,
        bytes: u64,
    ) -> c_int;
    pub fn vx_fill_u32(ctx: *mut VxCtx, dst: *mut VxBuf, dst_offset: u64, value: u32, count: u64) -> c_int;
    pub fn vx_sync(ctx: *mut VxCtx) -> c_int;
    pub fn vx_set_cancel_flag(ctx: *mut VxCtx, flag: *const u32) -> c_int;
    pub fn vx_graph_begin(ctx: *mut VxCtx) -> c_int;
    pub fn vx_graph_end(ctx: *mut VxCtx, out: *mut *mut VxGraph) -> c_int;
    pub fn vx_graph_launch(ctx: *mut VxCtx, graph: *mut VxGraph) -> c_int;
    pub fn vx_graph_free(ctx: *mut VxCtx, graph: *mut VxGraph) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxProfEntry {
    pub name: [c_char; 64],
    pub total_ms: f64,
    pub calls: u64,
    pub avg_ms: f64,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_prof_enable(ctx: *mut VxCtx, enabled: c_int) -> c_int;
    pub fn vx_prof_reset(ctx: *mut VxCtx) -> c_int;
    pub fn vx_prof_snapshot(ctx: *mut VxCtx, out: *mut VxProfEntry, cap: u32, count: *mut u32) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxTensorInfo {
    pub name: [c_char; 96],
    pub ggml_type: u32,
    pub n_dims: u32,
    pub dims: [u64; 4],
    pub offset: u64,
    pub bytes: u64,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_model_upload(
        ctx: *mut VxCtx,
        data: *const c_void,
        bytes: u64,
        tensors: *const VxTensorInfo,
        n_tensors: u32,
        out: *mut *mut VxModel,
    ) -> c_int;
    pub fn vx_model_free(ctx: *mut VxCtx, model: *mut VxModel) -> c_int;
    pub fn vx_model_tensor_count(model: *const VxModel) -> u32;
    pub fn vx_model_tensor_at(model: *const VxModel, index: u32, out: *mut VxTensorInfo) -> c_int;
    pub fn vx_model_find(model: *const VxModel, name: *const c_char, out: *mut VxTensorInfo) -> c_int;
    pub fn vx_model_device_bytes(model: *const VxModel) -> u64;
    pub fn vx_dequant(
        ctx: *mut VxCtx,
        model: *const VxModel,
        weight_offset: u32,
        rows: u32,
        cols: u32,
        dtype: u32,
        out: *mut VxBuf,
    ) -> c_int;
    pub fn vx_embedding(
        ctx: *mut VxCtx,
        model: *const VxModel,
        hidden: *mut VxBuf,
        pc: *const VxEmbeddingPush,
    ) -> c_int;
    pub fn vx_embedding_devtok(
        ctx: *mut VxCtx,
        model: *const VxModel,
        hidden: *mut VxBuf,
        tokens: *const VxBuf,
        position: *const VxBuf,
        pc: *const VxEmbeddingPush,
    ) -> c_int;
    pub fn vx_rmsnorm(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxRmsPush,
    ) -> c_int;
    pub fn vx_residual_rmsnorm(
        ctx: *mut VxCtx,
        model: *const VxModel,
        hidden: *mut VxBuf,
        branch: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxResidualRmsPush,
    ) -> c_int;
    pub fn vx_matvec(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxMatvecPush,
    ) -> c_int;
    pub fn vx_qkv_matvec(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        q: *mut VxBuf,
        k: *mut VxBuf,
        v: *mut VxBuf,
        pc: *const VxQkvPush,
    ) -> c_int;
    pub fn vx_matvec_swiglu(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxSwigluPush,
    ) -> c_int;
    pub fn vx_rope(
        ctx: *mut VxCtx,
        model: *const VxModel,
        q: *mut VxBuf,
        k: *mut VxBuf,
        pc: *const VxRopePush,
    ) -> c_int;
    pub fn vx_rope_devpos(
        ctx: *mut VxCtx,
        model: *const VxModel,
        q: *mut VxBuf,
        k: *mut VxBuf,
        position: *const VxBuf,
        pc: *const VxRopePush,
    ) -> c_int;
    pub fn vx_store_kv(
        ctx: *mut VxCtx,
        k: *const VxBuf,
        v: *const VxBuf,
        k_cache: *mut VxBuf,
        v_cache: *mut VxBuf,
        pc: *const VxStoreKvPush,
    ) -> c_int;
    pub fn vx_store_kv_devpos(
        ctx: *mut VxCtx,
        k: *const VxBuf,
        v: *const VxBuf,
        k_cache: *mut VxBuf,
        v_cache: *mut VxBuf,
        position: *const VxBuf,
        pc: *const VxStoreKvPush,
    ) -> c_int;
    pub fn vx_attn_scores(
        ctx: *mut VxCtx,
        q: *const VxBuf,
        k_cache: *const VxBuf,
        scores: *mut VxBuf,
        pc: *const VxAttentionPush,
    ) -> c_int;
    pub fn vx_attn_scores_devpos(
        ctx: *mut VxCtx,
        q: *const VxBuf,
        k_cache: *const VxBuf,
        scores: *mut VxBuf,
        position: *const VxBuf,
        pc: *const VxAttentionPush,
    ) -> c_int;
    pub fn vx_softmax(ctx: *mut VxCtx, scores: *mut VxBuf, heads: u32, pc: *const VxSoftmaxPush) -> c_int;
    pub fn vx_softmax_devpos(
        ctx: *mut VxCtx,
        scores: *mut VxBuf,
        heads: u32,
        position: *const VxBuf,
        pc: *const VxSoftmaxPush,
    ) -> c_int;
    pub fn vx_attn_values(
        ctx: *mut VxCtx,
        scores: *const VxBuf,
        v_cache: *const VxBuf,
        out: *mut VxBuf,
        pc: *const VxAttentionPush,
    ) -> c_int;
    pub fn vx_attn_values_devpos(
        ctx: *mut VxCtx,
        scores: *const VxBuf,
        v_cache: *const VxBuf,
        out: *mut VxBuf,
        position: *const VxBuf,
        pc: *const VxAttentionPush,
    ) -> c_int;
    pub fn vx_linear_bias(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxLinearBiasPush,
    ) -> c_int;
    pub fn vx_fusion_linear(
        ctx: *mut VxCtx,
        model: *const VxModel,
        left: *const VxBuf,
        right: *const VxBuf,
        y: *mut VxBuf,
        snapshot: *mut VxBuf,
        pc: *const VxFusionPush,
    ) -> c_int;
    pub fn vx_seq_linear_bias(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxSeqLinearPush,
    ) -> c_int;
    pub fn vx_seq_qkv(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        q: *mut VxBuf,
        k: *mut VxBuf,
        v: *mut VxBuf,
        pc: *const VxSeqQkvPush,
    ) -> c_int;
    pub fn vx_seq_swiglu(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxSeqSwigluPush,
    ) -> c_int;
    pub fn vx_seq_silu_mul(ctx: *mut VxCtx, gate: *mut VxBuf, up: *const VxBuf, n: u32) -> c_int;
    pub fn vx_seq_rmsnorm(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxSeqRmsPush,
    ) -> c_int;
    pub fn vx_seq_residual_rmsnorm(
        ctx: *mut VxCtx,
        model: *const VxModel,
        hidden: *mut VxBuf,
        branch: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxSeqResidualRmsPush,
    ) -> c_int;
    pub fn vx_seq_rope(
        ctx: *mut VxCtx,
        model: *const VxModel,
        q: *mut VxBuf,
        k: *mut VxBuf,
        pc: *const VxSeqRopePush,
    ) -> c_int;
    pub fn vx_seq_rope_at(
        ctx: *mut VxCtx,
        model: *const VxModel,
        q: *mut VxBuf,
        k: *mut VxBuf,
        position_base: u32,
        pc: *const VxSeqRopePush,
    ) -> c_int;
    pub fn vx_dense_attn_scores(
        ctx: *mut VxCtx,
        q: *const VxBuf,
        k: *const VxBuf,
        scores: *mut VxBuf,
        pc: *const VxDenseScoresPush,
    ) -> c_int;
    pub fn vx_dense_softmax(ctx: *mut VxCtx, scores: *mut VxBuf, pc: *const VxDenseSoftmaxPush) -> c_int;
    pub fn vx_dense_attn_values(
        ctx: *mut VxCtx,
        scores: *const VxBuf,
        v: *const VxBuf,
        out: *mut VxBuf,
        pc: *const VxDenseValuesPush,
    ) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxFusedQkvArgs {
    pub norm_offset: u32,
    pub eps: f32,
    pub q_weight_offset: u32,
    pub k_weight_offset: u32,
    pub v_weight_offset: u32,
    pub q_rows: u32,
    pub kv_rows: u32,
    pub cols: u32,
    pub dtype: u32,
    pub factor_offset: u32,
    pub head_dim: u32,
    pub rope_theta: f32,
    pub scaling_factor: f32,
    pub layer: u32,
    pub context: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_fused_qkv_rope_store(
        ctx: *mut VxCtx,
        model: *const VxModel,
        hidden: *const VxBuf,
        q: *mut VxBuf,
        k: *mut VxBuf,
        v: *mut VxBuf,
        k_cache: *mut VxBuf,
        v_cache: *mut VxBuf,
        position: *const VxBuf,
        a: *const VxFusedQkvArgs,
    ) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxFusedAttnArgs {
    pub layer: u32,
    pub context: u32,
    pub head_dim: u32,
    pub q_heads: u32,
    pub kv_heads: u32,
    pub splits: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_fused_attention_scratch_bytes(a: *const VxFusedAttnArgs) -> u64;
    pub fn vx_fused_attention(
        ctx: *mut VxCtx,
        q: *const VxBuf,
        k_cache: *const VxBuf,
        v_cache: *const VxBuf,
        out: *mut VxBuf,
        scratch: *mut VxBuf,
        position: *const VxBuf,
        a: *const VxFusedAttnArgs,
    ) -> c_int;
    pub fn vx_fused_attention_noalloc(
        ctx: *mut VxCtx,
        q: *const VxBuf,
        k_cache: *const VxBuf,
        v_cache: *const VxBuf,
        out: *mut VxBuf,
        position: *const VxBuf,
        a: *const VxFusedAttnArgs,
    ) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxFusedResidualArgs {
    pub weight_offset: u32,
    pub rows: u32,
    pub cols: u32,
    pub dtype: u32,
    pub scale: f32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_fused_matvec_residual(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        hidden: *mut VxBuf,
        branch: *mut VxBuf,
        a: *const VxFusedResidualArgs,
    ) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxFusedSwigluArgs {
    pub norm_offset: u32,
    pub eps: f32,
    pub gate_weight_offset: u32,
    pub up_weight_offset: u32,
    pub rows: u32,
    pub cols: u32,
    pub dtype: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_fused_rms_swiglu(
        ctx: *mut VxCtx,
        model: *const VxModel,
        hidden: *const VxBuf,
        y: *mut VxBuf,
        a: *const VxFusedSwigluArgs,
    ) -> c_int;
    pub fn vx_diag_stream_read(
        ctx: *mut VxCtx,
        src: *const VxBuf,
        offset: u64,
        bytes: u64,
        sink: *mut VxBuf,
        blocks: u32,
        unroll: u32,
    ) -> c_int;
    pub fn vx_diag_stream_copy(
        ctx: *mut VxCtx,
        dst: *mut VxBuf,
        src: *const VxBuf,
        bytes: u64,
        blocks: u32,
    ) -> c_int;
    pub fn vx_diag_timeline_arm(ctx: *mut VxCtx, waves: u64) -> c_int;
    pub fn vx_diag_timeline_read(
        ctx: *mut VxCtx,
        launches: *mut u64,
        max_launches: u64,
        ticks: *mut u64,
        max_waves: u64,
        n_launches: *mut u64,
        n_waves: *mut u64,
    ) -> c_int;
    pub fn vx_gguf_open(path: *const c_char, out: *mut *mut VxGguf) -> c_int;
    pub fn vx_gguf_close(g: *mut VxGguf) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxGgufSummary {
    pub version: u32,
    pub tensor_count: u64,
    pub metadata_count: u64,
    pub alignment: u64,
    pub data_offset: u64,
    pub file_bytes: u64,
    pub tensor_bytes: u64,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_gguf_summary_get(g: *const VxGguf, out: *mut VxGgufSummary) -> c_int;
    pub fn vx_gguf_tensor_at(g: *const VxGguf, index: u32, out: *mut VxTensorInfo) -> c_int;
    pub fn vx_gguf_find(g: *const VxGguf, name: *const c_char, out: *mut VxTensorInfo) -> c_int;
    pub fn vx_gguf_meta(g: *const VxGguf, key: *const c_char, out: *mut c_char, cap: u32) -> c_int;
    pub fn vx_gguf_primary_format(g: *const VxGguf, dtype_out: *mut u32) -> c_int;
    pub fn vx_model_upload_gguf(ctx: *mut VxCtx, g: *const VxGguf, out: *mut *mut VxModel) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxBaselmConfig {
    pub context_length: u32,
    pub active_context_length: u32,
    pub embedding_length: u32,
    pub block_count: u32,
    pub feed_forward_length: u32,
    pub vocab_size: u32,
    pub head_count: u32,
    pub head_count_kv: u32,
    pub head_dim: u32,
    pub kv_dim: u32,
    pub rms_epsilon: f32,
    pub rope_theta: f32,
    pub rope_dimension_count: u32,
    pub rope_original_context_length: u32,
    pub rope_longrope: u32,
    pub embedding_scale: f32,
    pub residual_scale: f32,
    pub logit_scale: f32,
    pub tied_output: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_baselm_config_from_gguf(
        g: *const VxGguf,
        active_context_length: u32,
        out: *mut VxBaselmConfig,
    ) -> c_int;
    pub fn vx_baselm_rope_scaling_factor(cfg: *const VxBaselmConfig) -> f32;
    pub fn vx_baselm_kv_cache_bytes(cfg: *const VxBaselmConfig) -> u64;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxBaselmOptions {
    pub exec_mode: u32,
    pub strict_geometry: u32,
    pub attn_splits: u32,
    pub prefill_schedule: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_baselm_create(
        ctx: *mut VxCtx,
        model: *const VxModel,
        cfg: *const VxBaselmConfig,
        opt: *const VxBaselmOptions,
        out: *mut *mut VxBaselm,
    ) -> c_int;
    pub fn vx_baselm_destroy(eng: *mut VxBaselm) -> c_int;
    pub fn vx_baselm_reset(eng: *mut VxBaselm) -> c_int;
    pub fn vx_baselm_position(eng: *const VxBaselm) -> u32;
    pub fn vx_baselm_set_position(eng: *mut VxBaselm, position: u32) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxTopLogit {
    pub token_id: u32,
    pub logit: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxStepResult {
    pub position: u32,
    pub elapsed_ms: f64,
    pub final_hidden_checksum: f64,
    pub final_hidden_l2: f64,
    pub n_top: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_top_k_logits(
        logits: *const f32,
        n: u32,
        k: u32,
        out: *mut VxTopLogit,
        n_out: *mut u32,
    ) -> c_int;
    pub fn vx_baselm_decode_token(
        eng: *mut VxBaselm,
        token_id: u32,
        top_k: u32,
        res: *mut VxStepResult,
        top: *mut VxTopLogit,
    ) -> c_int;
    pub fn vx_baselm_decode_embedding(
        eng: *mut VxBaselm,
        embedding: *const f32,
        n: u32,
        top_k: u32,
        res: *mut VxStepResult,
        top: *mut VxTopLogit,
    ) -> c_int;
    pub fn vx_baselm_decode_token_gpu_only(
        eng: *mut VxBaselm,
        token_id: u32,
        position_out: *mut u32,
    ) -> c_int;
    pub fn vx_baselm_decode_embedding_gpu_only(
        eng: *mut VxBaselm,
        embedding: *const f32,
        n: u32,
        position_out: *mut u32,
    ) -> c_int;
    pub fn vx_baselm_decode_embedding_from_gpu_only(
        eng: *mut VxBaselm,
        source: *const VxBuf,
        position_out: *mut u32,
    ) -> c_int;
    pub fn vx_baselm_decode_tokens_gpu_only(eng: *mut VxBaselm, tokens: *const u32, n: u32) -> c_int;
    pub fn vx_baselm_prefill_tokens(
        eng: *mut VxBaselm,
        tokens: *const u32,
        n: u32,
        top_k_last: u32,
        res: *mut VxStepResult,
        top: *mut VxTopLogit,
    ) -> c_int;
    pub fn vx_baselm_prefill_tokens_batched(
        eng: *mut VxBaselm,
        tokens: *const u32,
        n: u32,
        top_k_last: u32,
        res: *mut VxStepResult,
        top: *mut VxTopLogit,
    ) -> c_int;
    pub fn vx_baselm_prefill_tokens_batched_gpu_only(eng: *mut VxBaselm, tokens: *const u32, n: u32) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxBaselmBenchmarkResult {
    pub iterations: u32,
    pub token_id: u32,
    pub mean_ms: f64,
    pub min_ms: f64,
    pub max_ms: f64,
    pub tokens_per_second: f64,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_baselm_benchmark(
        eng: *mut VxBaselm,
        token_id: u32,
        warmup: u32,
        iterations: u32,
        out: *mut VxBaselmBenchmarkResult,
    ) -> c_int;
    pub fn vx_baselm_buffer(eng: *mut VxBaselm, which: u32) -> *mut VxBuf;
    pub fn vx_baselm_profile_steps(
        eng: *mut VxBaselm,
        tokens: *const u32,
        n: u32,
        out: *mut VxProfEntry,
        cap: u32,
        count: *mut u32,
    ) -> c_int;
    pub fn vx_baselm_time_layer_kernel(eng: *mut VxBaselm, which: u32, reps: u32, avg_ms: *mut f64) -> c_int;
    pub fn vx_cfm_noise(ctx: *mut VxCtx, x: *mut VxBuf, pc: *const VxCfmNoisePush) -> c_int;
    pub fn vx_cfm_cfg_euler(
        ctx: *mut VxCtx,
        x: *mut VxBuf,
        positive: *const VxBuf,
        negative: *const VxBuf,
        pc: *const VxCfmEulerPush,
    ) -> c_int;
    pub fn vx_time_sinusoidal(ctx: *mut VxCtx, out: *mut VxBuf, pc: *const VxTimePush) -> c_int;
    pub fn vx_pack_locdit(
        ctx: *mut VxCtx,
        mu1: *const VxBuf,
        mu2: *const VxBuf,
        time: *const VxBuf,
        cond: *const VxBuf,
        x: *const VxBuf,
        hidden: *mut VxBuf,
        pc: *const VxPackLocditPush,
    ) -> c_int;
    pub fn vx_silu_inplace(ctx: *mut VxCtx, x: *mut VxBuf, n: u32) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxFsqPush {
    pub n: u32,
    pub scale: f32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_fsq_quantize(ctx: *mut VxCtx, latent: *mut VxBuf, pc: *const VxFsqPush) -> c_int;
    pub fn vx_add_vectors(ctx: *mut VxCtx, a: *mut VxBuf, b: *const VxBuf, n: u32) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxLocditConfig {
    pub hidden: u32,
    pub layers: u32,
    pub q_heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub ffn: u32,
    pub feat_dim: u32,
    pub patch: u32,
    pub n_mu: u32,
    pub n_cond: u32,
    pub cond_raw: u32,
    pub uncond_zero_cond: u32,
    pub rms_epsilon: f32,
    pub rope_theta: f32,
    pub rope_scaling: f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxCfmOptions {
    pub n_timesteps: u32,
    pub cfg_value: f32,
    pub temperature: f32,
    pub sway_sampling_coef: f32,
    pub seed: u64,
    pub use_cfg_zero_star: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxCfmResult {
    pub elapsed_ms: f64,
    pub n_timesteps: u32,
    pub estimator_calls: u32,
    pub zero_init_steps: u32,
    pub output_checksum: f64,
    pub output_l2: f64,
    pub output_min: f32,
    pub output_max: f32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_locdit_create(
        ctx: *mut VxCtx,
        model: *const VxModel,
        rope_model: *const VxModel,
        rope_factor_offset: u32,
        cfg: *const VxLocditConfig,
        strict_geometry: u32,
        out: *mut *mut VxLocdit,
    ) -> c_int;
    pub fn vx_locdit_destroy(loc: *mut VxLocdit) -> c_int;
    pub fn vx_locdit_estimate(
        loc: *mut VxLocdit,
        x: *const f32,
        cond: *const f32,
        mu: *const f32,
        t: f32,
        dt: f32,
        out: *mut f32,
    ) -> c_int;
    pub fn vx_locdit_cfm_solve(
        loc: *mut VxLocdit,
        cond: *const f32,
        mu: *const f32,
        opt: *const VxCfmOptions,
        initial_x: *const f32,
        out_patch: *mut f32,
        res: *mut VxCfmResult,
    ) -> c_int;
    pub fn vx_locdit_cfm_solve_from_model_hiddens(
        loc: *mut VxLocdit,
        current_lm: *const VxBuf,
        residual_output: *const VxBuf,
        cond: *const f32,
        opt: *const VxCfmOptions,
        initial_x: *const f32,
        out_patch: *mut f32,
        res: *mut VxCfmResult,
    ) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxAcousticConfig {
    pub model_version: f32,
    pub residual_block_count: u32,
    pub embedding_length: u32,
    pub feed_forward_length: u32,
    pub head_count: u32,
    pub head_count_kv: u32,
    pub head_dim: u32,
    pub kv_dim: u32,
    pub no_rope: u32,
    pub active_context_length: u32,
    pub rms_epsilon: f32,
    pub residual_scale: f32,
    pub fsq_latent_dim: u32,
    pub fsq_scale: f32,
    pub fusion_input_dim: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_acoustic_config_from_gguf(
        g: *const VxGguf,
        base: *const VxBaselmConfig,
        active_context_length: u32,
        out: *mut VxAcousticConfig,
    ) -> c_int;
    pub fn vx_acoustic_kv_cache_bytes(cfg: *const VxAcousticConfig) -> u64;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxResidualOptions {
    pub exec_mode: u32,
    pub strict_geometry: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxFsqResult {
    pub elapsed_ms: f64,
    pub output_checksum: f64,
    pub output_l2: f64,
    pub latent_checksum: f64,
    pub latent_l2: f64,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxResidualStepResult {
    pub position: u32,
    pub fsq_applied: u32,
    pub elapsed_ms: f64,
    pub fsq_checksum: f64,
    pub fsq_l2: f64,
    pub fused_input_checksum: f64,
    pub fused_input_l2: f64,
    pub residual_hidden_checksum: f64,
    pub residual_hidden_l2: f64,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxResidualGpuStep {
    pub position: u32,
    pub fsq_applied: u32,
    pub elapsed_ms: f64,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxResidualBenchmarkResult {
    pub iterations: u32,
    pub mean_ms: f64,
    pub min_ms: f64,
    pub max_ms: f64,
    pub steps_per_second: f64,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxStopPrediction {
    pub stop: u32,
    pub continue_logit: f32,
    pub stop_logit: f32,
    pub elapsed_ms: f64,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_residual_create(
        ctx: *mut VxCtx,
        acoustic: *const VxModel,
        cfg: *const VxAcousticConfig,
        opt: *const VxResidualOptions,
        out: *mut *mut VxResidual,
    ) -> c_int;
    pub fn vx_residual_destroy(eng: *mut VxResidual) -> c_int;
    pub fn vx_residual_position(eng: *const VxResidual) -> u32;
    pub fn vx_residual_reset(eng: *mut VxResidual) -> c_int;
    pub fn vx_residual_allocated_bytes(eng: *const VxResidual) -> u64;
    pub fn vx_residual_buffer(eng: *mut VxResidual, which: u32) -> *mut VxBuf;
    pub fn vx_residual_fsq_only(
        eng: *mut VxResidual,
        base_hidden: *const f32,
        n: u32,
        out: *mut VxFsqResult,
    ) -> c_int;
    pub fn vx_residual_step(
        eng: *mut VxResidual,
        base_hidden: *const f32,
        current_embedding: *const f32,
        n: u32,
        out: *mut VxResidualStepResult,
    ) -> c_int;
    pub fn vx_residual_step_from_gpu_base(
        eng: *mut VxResidual,
        base_hidden: *const VxBuf,
        current_embedding: *const f32,
        n: u32,
        out: *mut VxResidualStepResult,
    ) -> c_int;
    pub fn vx_residual_step_from_gpu_base_and_embedding(
        eng: *mut VxResidual,
        base_hidden: *const VxBuf,
        current_embedding: *const VxBuf,
        out: *mut VxResidualStepResult,
    ) -> c_int;
    pub fn vx_residual_step_from_gpu_base_and_embedding_gpu_only(
        eng: *mut VxResidual,
        base_hidden: *const VxBuf,
        current_embedding: *const VxBuf,
        out: *mut VxResidualGpuStep,
    ) -> c_int;
    pub fn vx_residual_step_text_prefix_from_gpu_base(
        eng: *mut VxResidual,
        base_hidden: *const VxBuf,
        out: *mut VxResidualStepResult,
    ) -> c_int;
    pub fn vx_residual_step_text_prefix_from_gpu_base_gpu_only(
        eng: *mut VxResidual,
        base_hidden: *const VxBuf,
        out: *mut VxResidualGpuStep,
    ) -> c_int;
    pub fn vx_residual_benchmark(
        eng: *mut VxResidual,
        base_hidden: *const f32,
        current_embedding: *const f32,
        n: u32,
        warmup: u32,
        iterations: u32,
        out: *mut VxResidualBenchmarkResult,
    ) -> c_int;
    pub fn vx_residual_predict_stop_from_gpu_base(
        eng: *mut VxResidual,
        base_hidden: *const VxBuf,
        out: *mut VxStopPrediction,
    ) -> c_int;
    pub fn vx_residual_predict_stop_from_current_lm(
        eng: *mut VxResidual,
        out: *mut VxStopPrediction,
    ) -> c_int;
    pub fn vx_residual_prefill_text_from_gpu_rows(eng: *mut VxResidual, rows: *const VxBuf, n: u32) -> c_int;
    pub fn vx_prefill_text_cross_engine(
        base: *mut VxBaselm,
        eng: *mut VxResidual,
        tokens: *const u32,
        n: u32,
    ) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxVaeConvPush {
    pub weight_offset: u32,
    pub bias_offset: u32,
    pub in_channels: u32,
    pub out_channels: u32,
    pub in_length: u32,
    pub out_length: u32,
    pub kernel: u32,
    pub stride: u32,
    pub dilation: u32,
    pub groups: u32,
    pub left_pad: u32,
    pub weight_dtype: u32,
    pub bias_dtype: u32,
    pub has_bias: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxVaeConvtPush {
    pub weight_offset: u32,
    pub bias_offset: u32,
    pub in_channels: u32,
    pub out_channels: u32,
    pub in_length: u32,
    pub out_length: u32,
    pub kernel: u32,
    pub stride: u32,
    pub groups: u32,
    pub weight_dtype: u32,
    pub bias_dtype: u32,
    pub has_bias: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxVaeSnakePush {
    pub alpha_offset: u32,
    pub channels: u32,
    pub length: u32,
    pub dtype: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxVaeScalePush {
    pub scale_offset: u32,
    pub bias_offset: u32,
    pub channels: u32,
    pub length: u32,
    pub bucket: u32,
    pub buckets: u32,
    pub scale_dtype: u32,
    pub bias_dtype: u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxVaeGridPush {
    pub channels: u32,
    pub length: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_vae_conv1d(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxVaeConvPush,
    ) -> c_int;
    pub fn vx_vae_convtranspose1d(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxVaeConvtPush,
    ) -> c_int;
    pub fn vx_vae_snake(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *const VxBuf,
        y: *mut VxBuf,
        pc: *const VxVaeSnakePush,
    ) -> c_int;
    pub fn vx_vae_scale_bias(
        ctx: *mut VxCtx,
        model: *const VxModel,
        x: *mut VxBuf,
        pc: *const VxVaeScalePush,
    ) -> c_int;
    pub fn vx_vae_add(ctx: *mut VxCtx, a: *mut VxBuf, b: *const VxBuf, pc: *const VxVaeGridPush) -> c_int;
    pub fn vx_vae_tanh(ctx: *mut VxCtx, x: *mut VxBuf, n: u32) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxAudiovaeConfig {
    pub encoder_dim: u32,
    pub latent_dim: u32,
    pub decoder_dim: u32,
    pub sample_rate: u32,
    pub out_sample_rate: u32,
    pub encoder_rates: [u32; 4],
    pub decoder_rates: [u32; 6],
    pub encoder_hop: u32,
    pub decoder_hop: u32,
    pub patch_size: u32,
    pub input_samples_per_patch: u32,
    pub output_samples_per_patch: u32,
    pub sr_bin_boundaries: [u32; 3],
    pub decoder_sr_bucket: u32,
    pub depthwise: u32,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_audiovae_config_from_gguf(g: *const VxGguf, out: *mut VxAudiovaeConfig) -> c_int;
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct VxAudioDecodeStats {
    pub latent_frames: u32,
    pub latent_patches: u32,
    pub output_samples: u32,
    pub output_sample_rate: u32,
    pub duration_seconds: f64,
    pub checksum: f64,
    pub l2: f64,
    pub peak: f32,
    pub decode_ms: f64,
    pub scratch_bytes: u64,
}

#[link(name = "voxhip")]
extern "C" {
    pub fn vx_audiovae_create(
        ctx: *mut VxCtx,
        model: *const VxModel,
        cfg: *const VxAudiovaeConfig,
        strict_geometry: u32,
        out: *mut *mut VxAudiovae,
    ) -> c_int;
    pub fn vx_audiovae_destroy(vae: *mut VxAudiovae) -> c_int;
    pub fn vx_audiovae_scratch_bytes(vae: *const VxAudiovae) -> u64;
    pub fn vx_audiovae_decode_latents(
        vae: *mut VxAudiovae,
        frame_major: *const f32,
        n_values: u64,
        wave: *mut f32,
        wave_cap: u64,
        out: *mut VxAudioDecodeStats,
    ) -> c_int;
    pub fn vx_audiovae_decode_latents_gpu(
        vae: *mut VxAudiovae,
        frame_major: *const VxBuf,
        frames: u32,
        wave: *mut VxBuf,
    ) -> c_int;
}

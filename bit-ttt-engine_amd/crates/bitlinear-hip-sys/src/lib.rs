//! Raw bindings of libbitlinear_hip: every function, struct and constant of
//! `include/bitlinear.h` and `include/bitllama.h`, one to one (same names, same
//! argument order, C types mapped to their Rust equivalents), plus a safe
//! wrapper (`safe`) and, with the `candle` feature, the arm a maintainer adds to
//! the reference's `BitLinear::forward` (`crates/rust_engine/src/layers/bit_linear.rs:67-85`).
//!
//! Conventions of the C ABI: every call returns a status (`BTL_OK` or a
//! `BTL_ERR_*` code; `btl_last_error()` holds the thread's message), pointers are
//! device pointers unless a function says host, and `stream` is a
//! `hipStream_t` passed as `*mut c_void` (null: the default stream).
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_double, c_int, c_void};

pub mod safe;
#[cfg(feature = "candle")]
pub mod candle_arm;

// ---------------------------------------------------------------------------
// include/bitlinear.h
// ---------------------------------------------------------------------------

pub const BTL_VERSION: c_int = 1;

pub const BTL_OK: c_int = 0;
pub const BTL_ERR_SHAPE: c_int = 1;
pub const BTL_ERR_DTYPE: c_int = 2;
pub const BTL_ERR_LAYOUT: c_int = 3;
pub const BTL_ERR_DEVICE: c_int = 4;
pub const BTL_ERR_HIP: c_int = 5;
pub const BTL_ERR_ARG: c_int = 6;
pub const BTL_ERR_WORKSPACE: c_int = 7;
pub const BTL_ERR_FAULT: c_int = 8;

/// element types of activations and outputs
pub const BTL_F32: c_int = 0;
pub const BTL_BF16: c_int = 1;

/// arithmetic modes: the reference's fp32 order (cpu.rs, bit for bit: AVX2/FMA
/// lanes, or the sequential loop of a host without them) and W1.58-A8
pub const BTL_ACT_F32_REF: c_int = 0;
pub const BTL_ACT_I8: c_int = 1;
pub const BTL_ACT_F32_SEQ: c_int = 2;

/// `btl_packed_t`: the reference's PackedTensor (packing.rs:14-21) with its bytes
/// on the device: row-major [n, k] ternary weights, 4 per byte (code 01 = +1,
/// 10 = -1, 00 / 11 = 0, weight 4i + j in bits 2j..2j+1 of byte i).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct btl_packed_t {
    pub data: *const u8,
    pub n: i64,
    pub k: i64,
    pub scale: f32,
}

extern "C" {
    pub fn btl_version() -> c_int;
    pub fn btl_last_error() -> *const c_char;
    pub fn btl_status_string(status: c_int) -> *const c_char;
    pub fn btl_init(device: c_int) -> c_int;
    pub fn btl_set_tuning(name: *const c_char, value: c_int) -> c_int;
    pub fn btl_get_tuning(name: *const c_char, value: *mut c_int) -> c_int;
    pub fn btl_check_faults(stream: *mut c_void) -> c_int;
    pub fn btl_last_gemm_form() -> *const c_char;

    pub fn btl_packed_bytes(n: i64, k: i64) -> i64;
    pub fn btl_pack_host(w: *const f32, n: i64, k: i64, out: *mut u8, scale: *mut f32) -> c_int;
    pub fn btl_unpack_host(data: *const u8, n: i64, k: i64, scale: f32, out: *mut f32) -> c_int;
    pub fn btl_pack_device(w: *const f32, n: i64, k: i64, out: *mut u8, scale: *mut f32, ws: *mut c_void,
                           ws_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn btl_pack_workspace_bytes(n: i64, k: i64) -> usize;
    pub fn btl_unpack_device(w: *const btl_packed_t, out: *mut f32, stream: *mut c_void) -> c_int;

    pub fn btl_quantize_act(x: *const c_void, xdtype: c_int, m: i64, k: i64, xq: *mut i8, xscale: *mut f32,
                            stream: *mut c_void) -> c_int;
    pub fn btl_linear(w: *const btl_packed_t, x: *const c_void, xdtype: c_int, m: i64, k: i64, y: *mut c_void,
                      ydtype: c_int, mode: c_int, acc_out: *mut i32, ws: *mut c_void, ws_bytes: usize,
                      stream: *mut c_void) -> c_int;
    pub fn btl_linear_noalloc(w: *const btl_packed_t, x: *const c_void, xdtype: c_int, m: i64, k: i64,
                              y: *mut c_void, ydtype: c_int, mode: c_int, acc_out: *mut i32,
                              stream: *mut c_void) -> c_int;
    pub fn btl_linear_i8(w: *const btl_packed_t, xq: *const i8, xscale: *const f32, m: i64, k: i64,
                         y: *mut c_void, ydtype: c_int, acc_out: *mut i32, ws: *mut c_void, ws_bytes: usize,
                         stream: *mut c_void) -> c_int;
    pub fn btl_linear_group(w: *const *const btl_packed_t, y: *const *mut c_void, count: c_int, x: *const c_void,
                            xdtype: c_int, m: i64, k: i64, ydtype: c_int, ws: *mut c_void, ws_bytes: usize,
                            stream: *mut c_void) -> c_int;
    pub fn btl_linear_group_mode(w: *const *const btl_packed_t, y: *const *mut c_void, count: c_int,
                                 x: *const c_void, xdtype: c_int, m: i64, k: i64, ydtype: c_int, mode: c_int,
                                 ws: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn btl_quantize_act_op(x: *const c_void, xdtype: c_int, m: i64, k: i64, xq: *mut i8, xscale: *mut f32,
                               stream: *mut c_void) -> c_int;
    pub fn btl_linear_i8_op(w: *const *const btl_packed_t, y: *const *mut c_void, acc_out: *const *mut i32,
                            count: c_int, xq: *const i8, xscale: *const f32, m: i64, k: i64, ydtype: c_int,
                            stream: *mut c_void) -> c_int;
    pub fn btl_rmsnorm_linear_group(w: *const *const btl_packed_t, y: *const *mut c_void, count: c_int,
                                    x: *const c_void, xdtype: c_int, g: *const f32, eps: f32, m: i64, k: i64,
                                    ydtype: c_int, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn btl_swiglu_linear_group(w: *const *const btl_packed_t, y: *const *mut c_void, count: c_int,
                                   gate: *const c_void, up: *const c_void, xdtype: c_int, m: i64, k: i64,
                                   ydtype: c_int, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> c_int;

    // multi-base adaptive format (adaptive_linear.rs)
    pub fn btl_adaptive_split(packed: *const u8, n: i64, k: i64, nb: c_int, out: *const *mut u8,
                              stream: *mut c_void) -> c_int;
    pub fn btl_adaptive_reconstruct(packed: *const u8, scales: *const f32, nb: c_int, n: i64, k: i64,
                                    out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn btl_adaptive_linear(bases: *const *const btl_packed_t, nb: c_int, x: *const c_void, xdtype: c_int,
                               m: i64, k: i64, y: *mut c_void, ydtype: c_int, ws: *mut c_void, ws_bytes: usize,
                               stream: *mut c_void) -> c_int;
    pub fn btl_adaptive_workspace_bytes(m: i64, n: i64, k: i64, nb: c_int) -> usize;

    pub fn btl_workspace_bytes(m: i64, n: i64, k: i64, mode: c_int) -> usize;
    pub fn btl_workspace_clear(ws: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> c_int;
}

// ---------------------------------------------------------------------------
// include/bitllama.h
// ---------------------------------------------------------------------------

/// `btl_kv_q8_t`: one layer's Q8 KV cache (QuantizedKVCache, kv_cache.rs:14-22),
/// device arrays k, v [n_kv_heads, max_seq, head_dim] u8 and k_scale, v_scale
/// [n_kv_heads, max_seq] f32.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct btl_kv_q8_t {
    pub k: *mut u8,
    pub v: *mut u8,
    pub k_scale: *mut f32,
    pub v_scale: *mut f32,
    pub n_kv_heads: i64,
    pub max_seq: i64,
    pub head_dim: i64,
}

/// `btl_stream_layer_t`: the seven projections of one decoder layer for the
/// persistent decode stream (btl_stream_*).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct btl_stream_layer_t {
    pub q: btl_packed_t,
    pub k: btl_packed_t,
    pub v: btl_packed_t,
    pub o: btl_packed_t,
    pub gate: btl_packed_t,
    pub up: btl_packed_t,
    pub down: btl_packed_t,
}

extern "C" {
    pub fn btl_rope_table(theta: c_double, head_dim: i64, max_seq: i64, cos_out: *mut f32, sin_out: *mut f32)
                          -> c_int;
    pub fn btl_rope_kv_append(q: *const f32, k: *const f32, v: *const f32, m: i64, n_heads: i64,
                              cache: *const btl_kv_q8_t, pos: i64, d_pos: *const i32, rope_cos: *const f32,
                              rope_sin: *const f32, q_out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn btl_attention_workspace_bytes(m: i64, n_heads: i64, cache: *const btl_kv_q8_t) -> usize;
    pub fn btl_attention(q: *const f32, m: i64, n_heads: i64, cache: *const btl_kv_q8_t, pos: i64,
                         d_pos: *const i32, out: *mut f32, ws: *mut c_void, ws_bytes: usize,
                         stream: *mut c_void) -> c_int;
    pub fn btl_rope_append_attention(q: *const f32, k: *const f32, v: *const f32, m: i64, n_heads: i64,
                                     cache: *const btl_kv_q8_t, pos: i64, d_pos: *const i32,
                                     rope_cos: *const f32, rope_sin: *const f32, out: *mut f32, ws: *mut c_void,
                                     ws_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn btl_embedding(table: *const c_void, dtype: c_int, vocab: i64, dim: i64, ids: *const i32, m: i64,
                         out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn btl_greedy_next(logits: *const f32, n: i64, next_id: *mut i32, d_pos: *mut i32, log: *mut i32,
                           log_len: i64, stream: *mut c_void) -> c_int;
    pub fn btl_add_rmsnorm(h: *const f32, delta: *const f32, h_out: *mut f32, g: *const f32, eps: f32, m: i64,
                           k: i64, y: *mut f32, stream: *mut c_void) -> c_int;
    pub fn btl_swiglu(gate: *const f32, up: *const f32, count: i64, out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn btl_dense_linear(w: *const c_void, wdtype: c_int, n: i64, k: i64, x: *const f32, m: i64, y: *mut f32,
                            stream: *mut c_void) -> c_int;
    pub fn btl_add_rmsnorm_linear_group(w: *const *const btl_packed_t, y: *const *mut c_void, count: c_int,
                                        h: *const f32, delta: *const f32, h_out: *mut f32, g: *const f32,
                                        eps: f32, m: i64, k: i64, ydtype: c_int, ws: *mut c_void,
                                        ws_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn btl_add_rmsnorm_linear_group_ref(w: *const *const btl_packed_t, y: *const *mut c_void, count: c_int,
                                            h: *const f32, delta: *const f32, h_out: *mut f32, g: *const f32,
                                            eps: f32, m: i64, k: i64, stream: *mut c_void) -> c_int;
    pub fn btl_linear_residual(w: *const btl_packed_t, x: *const c_void, xdtype: c_int, m: i64, k: i64,
                               resid: *const f32, y: *mut f32, ws: *mut c_void, ws_bytes: usize,
                               stream: *mut c_void) -> c_int;
    pub fn btl_add_rmsnorm_swiglu(w_gate: *const btl_packed_t, w_up: *const btl_packed_t, h: *const f32,
                                  delta: *const f32, h_out: *mut f32, g: *const f32, eps: f32, m: i64, k: i64,
                                  out: *mut f32, ws: *mut c_void, ws_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn btl_add_rmsnorm_swiglu_workspace_bytes(m: i64, n: i64, k: i64) -> usize;

    pub fn btl_stream_create(layers: *const btl_stream_layer_t, n_layers: c_int, plan: *mut *mut c_void) -> c_int;
    pub fn btl_stream_stage_words(plan: *const c_void) -> usize;
    pub fn btl_stream_run(plan: *mut c_void, x: *const c_void, y: *mut c_void, stage_out: *mut c_void,
                          stream: *mut c_void) -> c_int;
    pub fn btl_stream_destroy(plan: *mut c_void) -> c_int;
}

// ---------------------------------------------------------------------------
// the HIP runtime calls the safe wrapper needs (libamdhip64)
// ---------------------------------------------------------------------------

pub type hipError_t = c_int;
pub type hipStream_t = *mut c_void;
pub const HIP_SUCCESS: hipError_t = 0;
pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

extern "C" {
    pub fn hipSetDevice(device: c_int) -> hipError_t;
    pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> hipError_t;
    pub fn hipFree(ptr: *mut c_void) -> hipError_t;
    pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> hipError_t;
    pub fn hipMemcpyAsync(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int, stream: hipStream_t)
                          -> hipError_t;
    pub fn hipStreamCreate(stream: *mut hipStream_t) -> hipError_t;
    pub fn hipStreamDestroy(stream: hipStream_t) -> hipError_t;
    pub fn hipStreamSynchronize(stream: hipStream_t) -> hipError_t;
    pub fn hipGetErrorString(err: hipError_t) -> *const c_char;
}

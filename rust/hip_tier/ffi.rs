//! Raw bindings to include/wave_hip_attn.h.
use std::os::raw::{c_char, c_int, c_void};

#[repr(C)]
#[derive(Clone, Copy)]
pub struct WhaLayout { pub b: i32, pub h: i32, pub t: i32, pub d: i32,
                       pub stride_b: i64, pub stride_h: i64, pub stride_t: i64 }

#[repr(C)] pub struct WhaWaveShape { pub b: i32, pub t: i32, pub n_embd: i32, pub n_head: i32, pub content_dim: i32 }
#[repr(C)] pub struct WhaWaveWeights { pub harmonic_raw: *const f32, pub proj_w: *const f32, pub proj_b: *const f32,
                                       pub v_w: *const f32, pub v_b: *const f32, pub out_w: *const f32, pub out_b: *const f32 }
#[repr(C)] pub struct WhaWaveCache { pub proj: *mut f32, pub values: *mut f32, pub feat: *mut f32, pub phase: *mut f32,
                                     pub bucket: *mut i32, pub merged: *mut f32, pub lse: *mut f32 }
#[repr(C)] pub struct WhaWaveGrads { pub d_x: *mut f32, pub d_harmonic_raw: *mut f32, pub d_proj_w: *mut f32,
                                     pub d_proj_b: *mut f32, pub d_v_w: *mut f32, pub d_v_b: *mut f32,
                                     pub d_out_w: *mut f32, pub d_out_b: *mut f32 }
#[repr(C)] pub struct WhaWaveKvCache { pub cs: *mut f32, pub bucket: *mut i32, pub phase: *mut f32,
                                       pub values: *mut f32, pub capacity: i32 }

extern "C" {
    pub fn wha_last_error() -> *const c_char;
    pub fn wha_version() -> *const c_char;
    pub fn wha_attn_fwd(q: *const f32, k: *const f32, v: *const f32, o: *mut f32, lse: *mut f32,
                        layout: *const WhaLayout, scale: f32, stream: *mut c_void) -> c_int;
    pub fn wha_attn_bwd_workspace_size(layout: *const WhaLayout) -> usize;
    pub fn wha_attn_bwd(q: *const f32, k: *const f32, v: *const f32, o: *const f32, d_o: *const f32,
                        lse: *const f32, dq: *mut f32, dk: *mut f32, dv: *mut f32,
                        workspace: *mut c_void, workspace_bytes: usize,
                        layout: *const WhaLayout, scale: f32, stream: *mut c_void) -> c_int;
    pub fn wha_attn_scores_size(layout: *const WhaLayout) -> usize;
    pub fn wha_attn_fwd_keep(q: *const f32, k: *const f32, v: *const f32, o: *mut f32, lse: *mut f32,
                             scores: *mut f32, layout: *const WhaLayout, scale: f32, stream: *mut c_void) -> c_int;
    pub fn wha_attn_bwd_kept(q: *const f32, k: *const f32, v: *const f32, o: *const f32, d_o: *const f32,
                             lse: *const f32, scores: *const f32, dq: *mut f32, dk: *mut f32, dv: *mut f32,
                             workspace: *mut c_void, workspace_bytes: usize,
                             layout: *const WhaLayout, scale: f32, stream: *mut c_void) -> c_int;
    pub fn wha_attn_bwd_from_probs_workspace_size(layout: *const WhaLayout) -> usize;
    pub fn wha_attn_bwd_from_probs(d_pre_proj: *const f32, q: *const f32, k: *const f32, v: *const f32,
                                   att: *const f32, dq: *mut f32, dk: *mut f32, dv: *mut f32,
                                   workspace: *mut c_void, workspace_bytes: usize,
                                   layout: *const WhaLayout, scale: f32, stream: *mut c_void) -> c_int;
    pub fn wha_decode_workspace_size(cache_layout: *const WhaLayout) -> usize;
    pub fn wha_decode_fwd(q: *const f32, k_cache: *const f32, v_cache: *const f32, o: *mut f32,
                          lse: *mut f32, workspace: *mut c_void, workspace_bytes: usize,
                          cache_layout: *const WhaLayout, scale: f32, stream: *mut c_void) -> c_int;
    pub fn wha_decode_fwd_noalloc(q: *const f32, k_cache: *const f32, v_cache: *const f32, o: *mut f32,
                                  lse: *mut f32, cache_layout: *const WhaLayout, scale: f32,
                                  stream: *mut c_void) -> c_int;
    pub fn wha_attn_probs_rows(q: *const f32, k: *const f32, lse: *const f32, rows: *const i32, n_rows: i32,
                               out: *mut f32, layout: *const WhaLayout, scale: f32, stream: *mut c_void) -> c_int;
    pub fn wha_linear_fwd(x: *const f32, ldx: i64, w: *const f32, b: *const f32, y: *mut f32, ldy: i64,
                          m: i64, n: i32, k: i32, stream: *mut c_void) -> c_int;
    pub fn wha_linear_bwd_dx(dy: *const f32, lddy: i64, w: *const f32, dx: *mut f32, lddx: i64,
                             m: i64, n: i32, k: i32, stream: *mut c_void) -> c_int;
    pub fn wha_linear_bwd_dw_workspace_size(m: i64, n: i32, k: i32) -> usize;
    pub fn wha_linear_bwd_dw(dy: *const f32, lddy: i64, x: *const f32, ldx: i64, dw: *mut f32, db: *mut f32,
                             m: i64, n: i32, k: i32, workspace: *mut c_void, workspace_bytes: usize,
                             stream: *mut c_void) -> c_int;
    pub fn wha_host_attention(x: *const f32, c_attn_w: *const f32, c_attn_b: *const f32, c_proj_w: *const f32,
                              c_proj_b: *const f32, t: i32, e: i32, n_head: i32, out: *mut f32) -> c_int;
    pub fn wha_host_attention_core_fwd(q: *const f32, k: *const f32, v: *const f32,
                                       t: i32, e: i32, n_head: i32, o: *mut f32) -> c_int;
    pub fn wha_host_attention_backward(d_pre_proj: *const f32, q: *const f32, k: *const f32,
                                       v: *const f32, att: *const f32, t: i32, e: i32, n_head: i32,
                                       dq: *mut f32, dk: *mut f32, dv: *mut f32) -> c_int;
    // wave attention (src/common/attn.rs) and its KV cache (src/common/kv_cache.rs)
    pub fn wha_wave_fwd_workspace_size(shape: *const WhaWaveShape) -> usize;
    pub fn wha_wave_fwd(x: *const f32, w: *const WhaWaveWeights, shape: *const WhaWaveShape, out: *mut f32,
                        cache: *const WhaWaveCache, workspace: *mut c_void, workspace_bytes: usize,
                        stream: *mut c_void) -> c_int;
    pub fn wha_wave_bwd_workspace_size(shape: *const WhaWaveShape) -> usize;
    pub fn wha_wave_bwd(x: *const f32, d_out: *const f32, w: *const WhaWaveWeights, shape: *const WhaWaveShape,
                        cache: *const WhaWaveCache, grads: *const WhaWaveGrads, workspace: *mut c_void,
                        workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn wha_wave_probs_rows(cache: *const WhaWaveCache, shape: *const WhaWaveShape, rows: *const i32,
                               n_rows: i32, out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn wha_wave_set_bucket_sparse(mode: c_int) -> c_int;
    pub fn wha_wave_kv_prefill_workspace_size(shape: *const WhaWaveShape) -> usize;
    pub fn wha_wave_kv_prefill(x: *const f32, w: *const WhaWaveWeights, shape: *const WhaWaveShape,
                               kv: *const WhaWaveKvCache, out: *mut f32, workspace: *mut c_void,
                               workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn wha_wave_kv_decode_workspace_size(shape: *const WhaWaveShape, capacity: i32) -> usize;
    pub fn wha_wave_kv_decode(x: *const f32, w: *const WhaWaveWeights, shape: *const WhaWaveShape,
                              kv: *const WhaWaveKvCache, lengths: *const i32, out: *mut f32,
                              workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn wha_host_wave_attention_forward(x: *const f32, w: *const WhaWaveWeights, t: i32, n_embd: i32,
                                           n_head: i32, content_dim: i32, out: *mut f32, phase_out: *mut f32) -> c_int;
    pub fn wha_host_wave_attention_backward(x: *const f32, d_attn_out: *const f32, w: *const WhaWaveWeights,
                                            t: i32, n_embd: i32, n_head: i32, content_dim: i32,
                                            g: *const WhaWaveGrads) -> c_int;
    pub fn wha_synth_normal(state: *mut u64, out: *mut f32, n: usize, stddev: f64, nthreads: c_int) -> c_int;
    pub fn wha_timing_enable(on: c_int) -> c_int;
    pub fn wha_timing_reset() -> c_int;
    pub fn wha_timing_read(kernel: *const c_char, total_ms: *mut f64, launches: *mut i64) -> c_int;
}

/// The reference's methods are infallible and panic on failure
/// (src/wgpu_tier/pipelines.rs:138); keep that contract.
pub fn check(rc: c_int, what: &str) {
    if rc != 0 {
        let msg = unsafe { std::ffi::CStr::from_ptr(wha_last_error()) }.to_string_lossy();
        panic!("{what} failed ({rc}): {msg}");
    }
}

//! HipBackend: ComputeBackend whose attention runs on MI355X (gfx950) kernels.
pub mod device;
pub mod ffi;
pub mod kv;
pub mod wave;

use crate::common::compute::{ComputeBackend, CpuBackend};
use crate::model::*;

pub struct HipBackend { cpu: CpuBackend }

impl HipBackend {
    pub fn new() -> Self { HipBackend { cpu: CpuBackend } }
}

fn flatten(rows: &[Vec<f32>]) -> Vec<f32> { rows.iter().flat_map(|r| r.iter().copied()).collect() }
fn unflatten(flat: Vec<f32>, e: usize) -> Vec<Vec<f32>> { flat.chunks(e).map(|c| c.to_vec()).collect() }

impl ComputeBackend for HipBackend {
    // src/common/compute.rs:42-43 = attention_cpu (:357-414) end to end on the GPU:
    // c_attn (:368-375), the causal core, c_proj (:411-413).
    fn attention(&self, w: &AttentionWeights, x: &[Vec<f32>]) -> Vec<Vec<f32>> {
        let (t, e) = (x.len(), x[0].len());
        let mut out = vec![0.0f32; t * e];
        ffi::check(unsafe { ffi::wha_host_attention(flatten(x).as_ptr(), flatten(&w.c_attn.w).as_ptr(),
                                                    w.c_attn.b.as_ptr(), flatten(&w.c_proj.w).as_ptr(),
                                                    w.c_proj.b.as_ptr(), t as i32, e as i32, w.n_head as i32,
                                                    out.as_mut_ptr()) }, "attention");
        unflatten(out, e)
    }

    // src/common/compute.rs:163-173 with CpuBackend's semantics (:286-314): att used as given.
    fn attention_backward(&self, d_pre_proj: &[Vec<f32>], q_all: &[Vec<f32>], k_all: &[Vec<f32>],
                          v_all: &[Vec<f32>], att_weights: &[Vec<Vec<f32>>], n_head: usize)
                          -> (Vec<Vec<f32>>, Vec<Vec<f32>>, Vec<Vec<f32>>) {
        let t = d_pre_proj.len();
        let e = d_pre_proj[0].len();
        let (d, q, k, v) = (flatten(d_pre_proj), flatten(q_all), flatten(k_all), flatten(v_all));
        let att: Vec<f32> = att_weights.iter().flat_map(|h| h.iter().flat_map(|r| r.iter().copied())).collect();
        let (mut dq, mut dk, mut dv) = (vec![0.0f32; t * e], vec![0.0f32; t * e], vec![0.0f32; t * e]);
        ffi::check(unsafe { ffi::wha_host_attention_backward(d.as_ptr(), q.as_ptr(), k.as_ptr(), v.as_ptr(),
                                                               att.as_ptr(), t as i32, e as i32, n_head as i32,
                                                               dq.as_mut_ptr(), dk.as_mut_ptr(), dv.as_mut_ptr()) },
                   "attention_backward");
        (unflatten(dq, e), unflatten(dk, e), unflatten(dv, e))
    }

    // everything else: the CPU backend, unchanged
    fn linear(&self, w: &[Vec<f32>], b: &[f32], x: &[f32]) -> Vec<f32> { self.cpu.linear(w, b, x) }
    fn linear_no_bias(&self, w: &[Vec<f32>], x: &[f32]) -> Vec<f32> { self.cpu.linear_no_bias(w, x) }
    fn layer_norm(&self, x: &[f32], w: &[f32], b: &[f32]) -> Vec<f32> { self.cpu.layer_norm(x, w, b) }
    fn kerr_ode(&self, w: &KerrWeights, x: &[f32]) -> Vec<f32> { self.cpu.kerr_ode(w, x) }
    fn maestro(&self, w: &MaestroWeights, x: &[f32]) -> Vec<f32> { self.cpu.maestro(w, x) }
    fn per_band_linear(&self, w: &PerBandLinearWeights, x: &[Vec<f32>]) -> Vec<Vec<f32>> { self.cpu.per_band_linear(w, x) }
    fn kerr_maestro_add(&self, w: &KerrMaestroAddWeights, x: &[Vec<f32>]) -> Vec<Vec<f32>> { self.cpu.kerr_maestro_add(w, x) }
    fn kerr_dual_maestro_add(&self, w: &KerrDualMaestroWeights, x: &[Vec<f32>]) -> Vec<Vec<f32>> { self.cpu.kerr_dual_maestro_add(w, x) }
    fn linear_backward_dx(&self, d_y: &[f32], w: &[Vec<f32>]) -> Vec<f32> { self.cpu.linear_backward_dx(d_y, w) }
    fn layer_norm_backward(&self, d_y: &[f32], x: &[f32], w: &[f32]) -> (Vec<f32>, Vec<f32>, Vec<f32>) { self.cpu.layer_norm_backward(d_y, x, w) }
    fn gelu_backward(&self, d_y: &[f32], x: &[f32]) -> Vec<f32> { self.cpu.gelu_backward(d_y, x) }
    fn linear_backward_dx_batch(&self, d_y: &[Vec<f32>], w: &[Vec<f32>]) -> Vec<Vec<f32>> { self.cpu.linear_backward_dx_batch(d_y, w) }
    fn outer_product_accum(&self, d_y: &[Vec<f32>], x: &[Vec<f32>], bias: bool) -> (Vec<Vec<f32>>, Vec<f32>) { self.cpu.outer_product_accum(d_y, x, bias) }
}

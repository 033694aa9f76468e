//! Wave attention (src/common/attn.rs:72-511) on the MI355X tier, host arrays in and out:
//! the drop-in for wave_attention_forward / _backward_full / _pathway, called from
//! src/cpu/forward.rs:113 and src/cpu/model_backward.rs:380-395.
use super::ffi::{self, WhaWaveGrads, WhaWaveWeights};
use crate::common::attn::{WaveAttnCache, WaveAttnGrads, WaveAttnHeadGrads, WaveAttnWeights};

/// WaveAttnWeights (attn.rs:17-46) packed into the ABI layout: per head the rows
/// phase_proj_w[0], phase_proj_w[1], content_proj_w[..] of proj_w, then v_proj and out_proj.
pub struct Packed { pub(crate) hraw: Vec<f32>, pub(crate) pw: Vec<f32>, pub(crate) pb: Vec<f32>,
                    pub(crate) vw: Vec<f32>, pub(crate) vb: Vec<f32>, pub(crate) ow: Vec<f32>,
                    pub(crate) ob: Vec<f32>, pub c: usize }
impl Packed {
    pub fn new(w: &WaveAttnWeights) -> Self {
        let c = w.heads[0].content_proj_w.len();
        let mut p = Packed { hraw: vec![], pw: vec![], pb: vec![], vw: vec![], vb: vec![],
                             ow: w.out_proj_w.concat(), ob: w.out_proj_b.clone(), c };
        for h in &w.heads {
            p.hraw.push(h.harmonic_raw);
            p.pw.extend(h.phase_proj_w.concat()); p.pw.extend(h.content_proj_w.concat());
            p.pb.extend(&h.phase_proj_b); p.pb.extend(&h.content_proj_b);
            p.vw.extend(h.v_proj_w.concat()); p.vb.extend(&h.v_proj_b);
        }
        p
    }
    fn abi(&self) -> WhaWaveWeights {
        WhaWaveWeights { harmonic_raw: self.hraw.as_ptr(), proj_w: self.pw.as_ptr(), proj_b: self.pb.as_ptr(),
                         v_w: self.vw.as_ptr(), v_b: self.vb.as_ptr(), out_w: self.ow.as_ptr(), out_b: self.ob.as_ptr() }
    }
}

/// wave_attention_forward(weights, x, n_bands, backend, _) (attn.rs:90-305): out and the phases.
pub fn wave_attention_forward(w: &WaveAttnWeights, x: &[Vec<f32>], n_bands: usize) -> (Vec<Vec<f32>>, Vec<Vec<f32>>) {
    let (t, e, h) = (x.len(), n_bands * 2, w.heads.len());
    let p = Packed::new(w);
    let (mut out, mut ph) = (vec![0.0f32; t * e], vec![0.0f32; h * t]);
    ffi::check(unsafe { ffi::wha_host_wave_attention_forward(x.concat().as_ptr(), &p.abi(), t as i32, e as i32,
                                                             h as i32, p.c as i32, out.as_mut_ptr(),
                                                             ph.as_mut_ptr()) }, "wave_attention_forward");
    (out.chunks(e).map(|r| r.to_vec()).collect(), ph.chunks(t).map(|r| r.to_vec()).collect())
}

/// wave_attention_backward_full (attn.rs:346-430): the ABI recomputes the cache from
/// `cache.normed` on the device; gradients come back in the packed layout and are
/// unpacked into the reference's per-head WaveAttnHeadGrads.
pub fn wave_attention_backward_full(w: &WaveAttnWeights, cache: &WaveAttnCache, d_attn_out: &[Vec<f32>]) -> WaveAttnGrads {
    let (t, e, h) = (d_attn_out.len(), cache.n_bands * 2, w.heads.len());
    let p = Packed::new(w);
    let (hd, pr) = (e / h, 2 + p.c);
    let mut d_x = vec![0.0f32; t * e];
    let (mut dh, mut dpw, mut dpb) = (vec![0.0f32; h], vec![0.0f32; h * pr * e], vec![0.0f32; h * pr]);
    let (mut dvw, mut dvb, mut dow, mut dob) = (vec![0.0f32; h * hd * hd], vec![0.0f32; h * hd], vec![0.0f32; e * e], vec![0.0f32; e]);
    let g = WhaWaveGrads { d_x: d_x.as_mut_ptr(), d_harmonic_raw: dh.as_mut_ptr(), d_proj_w: dpw.as_mut_ptr(),
                           d_proj_b: dpb.as_mut_ptr(), d_v_w: dvw.as_mut_ptr(), d_v_b: dvb.as_mut_ptr(),
                           d_out_w: dow.as_mut_ptr(), d_out_b: dob.as_mut_ptr() };
    ffi::check(unsafe { ffi::wha_host_wave_attention_backward(cache.normed.concat().as_ptr(), d_attn_out.concat().as_ptr(),
                                                              &p.abi(), t as i32, e as i32, h as i32, p.c as i32, &g) },
               "wave_attention_backward_full");
    unpack_grads(&d_x, &dh, &dpw, &dpb, &dvw, &dvb, &dow, &dob, t, e, h, p.c)
}

/// wave_attention_backward_pathway (attn.rs:432-511): the same call with every
/// weight-gradient pointer null; only d_normed comes back.
pub fn wave_attention_backward_pathway(w: &WaveAttnWeights, cache: &WaveAttnCache, d_attn_out: &[Vec<f32>]) -> Vec<Vec<f32>> {
    let (t, e, h) = (d_attn_out.len(), cache.n_bands * 2, w.heads.len());
    let p = Packed::new(w);
    let mut d_x = vec![0.0f32; t * e];
    let null = std::ptr::null_mut();
    let g = WhaWaveGrads { d_x: d_x.as_mut_ptr(), d_harmonic_raw: null, d_proj_w: null, d_proj_b: null,
                           d_v_w: null, d_v_b: null, d_out_w: null, d_out_b: null };
    ffi::check(unsafe { ffi::wha_host_wave_attention_backward(cache.normed.concat().as_ptr(), d_attn_out.concat().as_ptr(),
                                                              &p.abi(), t as i32, e as i32, h as i32, p.c as i32, &g) },
               "wave_attention_backward_pathway");
    d_x.chunks(e).map(|r| r.to_vec()).collect()
}

fn rows(flat: &[f32], width: usize) -> Vec<Vec<f32>> { flat.chunks(width).map(|r| r.to_vec()).collect() }

/// The packed gradients of the ABI (wha_wave_grads) into the reference's
/// per-head WaveAttnHeadGrads (attn.rs:318-326) and WaveAttnGrads (:331-336):
/// per head, rows 0..2 of d_proj_w are phase_proj_w, rows 2..2+c content_proj_w.
#[allow(clippy::too_many_arguments)]
fn unpack_grads(d_x: &[f32], dh: &[f32], dpw: &[f32], dpb: &[f32], dvw: &[f32], dvb: &[f32], dow: &[f32],
                dob: &[f32], _t: usize, e: usize, h: usize, c: usize) -> WaveAttnGrads {
    let (hd, pr) = (e / h, 2 + c);
    let heads = (0..h).map(|i| {
        let pw = &dpw[i * pr * e..(i + 1) * pr * e];
        let pb = &dpb[i * pr..(i + 1) * pr];
        WaveAttnHeadGrads {
            phase_proj_w: rows(&pw[..2 * e], e),
            phase_proj_b: pb[..2].to_vec(),
            v_proj_w: rows(&dvw[i * hd * hd..(i + 1) * hd * hd], hd),
            v_proj_b: dvb[i * hd..(i + 1) * hd].to_vec(),
            content_proj_w: rows(&pw[2 * e..], e),
            content_proj_b: pb[2..].to_vec(),
            d_harmonic_raw: dh[i],
        }
    }).collect();
    WaveAttnGrads { heads, out_proj_w: rows(dow, e), out_proj_b: dob.to_vec(), d_normed: rows(d_x, e) }
}

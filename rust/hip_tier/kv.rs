//! The attention half of the KV-cache serve path (src/common/kv_cache.rs:93-356,
//! driven by src/serve_tier/inference.rs:29-106) on the MI355X tier: one device
//! cache per layer for a batch of sequences, each with its own cached length.
//! The FFN, layer norms and sampling stay where they are.
use super::device::DeviceBuf;
use super::ffi::{self, WhaWaveKvCache, WhaWaveShape, WhaWaveWeights};
use super::wave::Packed;
use crate::common::attn::WaveAttnWeights;

/// One layer's attention weights resident on the device (packed per head as
/// wha_wave_weights describes), uploaded once instead of per token.
pub struct HipWaveLayer { bufs: [DeviceBuf; 7], n_embd: usize, n_head: usize, content_dim: usize }

impl HipWaveLayer {
    pub fn new(w: &WaveAttnWeights, n_embd: usize) -> Self {
        let p = Packed::new(w);
        let bufs = [DeviceBuf::from_slice(&p.hraw), DeviceBuf::from_slice(&p.pw), DeviceBuf::from_slice(&p.pb),
                    DeviceBuf::from_slice(&p.vw), DeviceBuf::from_slice(&p.vb), DeviceBuf::from_slice(&p.ow),
                    DeviceBuf::from_slice(&p.ob)];
        HipWaveLayer { bufs, n_embd, n_head: w.heads.len(), content_dim: p.c }
    }
    pub fn n_embd(&self) -> usize { self.n_embd }
    fn c(&self) -> WhaWaveWeights {
        let b = &self.bufs;
        WhaWaveWeights { harmonic_raw: b[0].ptr(), proj_w: b[1].ptr(), proj_b: b[2].ptr(), v_w: b[3].ptr(),
                         v_b: b[4].ptr(), out_w: b[5].ptr(), out_b: b[6].ptr() }
    }
    fn shape(&self, batch: usize, t: usize) -> WhaWaveShape {
        WhaWaveShape { b: batch as i32, t: t as i32, n_embd: self.n_embd as i32, n_head: self.n_head as i32,
                       content_dim: self.content_dim as i32 }
    }
}

/// HeadCache (kv_cache.rs:35-41) for every head of `batch` sequences:
/// cs [B][H][cap][2], bucket [B][H][cap] (i32), phase [B][H][cap],
/// values [B][H][cap][head_dim].
pub struct HipKvLayer { bufs: [DeviceBuf; 4], n_head: usize, head_dim: usize, capacity: usize,
                        lengths: Vec<i32> }

impl HipKvLayer {
    pub fn new(batch: usize, n_head: usize, head_dim: usize, capacity: usize) -> Self {
        let per = batch * n_head * capacity;
        HipKvLayer { bufs: [DeviceBuf::zeros(per * 2), DeviceBuf::zeros(per), DeviceBuf::zeros(per),
                            DeviceBuf::zeros(per * head_dim)],
                     n_head, head_dim, capacity, lengths: vec![0; batch] }
    }

    /// The cache as the ABI sees it, starting at sequence `seq` of the batch.
    fn slot(&self, seq: usize) -> WhaWaveKvCache {
        let per = self.n_head * self.capacity;
        WhaWaveKvCache { cs: self.bufs[0].at(seq * per * 2), bucket: self.bufs[1].at(seq * per) as *mut i32,
                         phase: self.bufs[2].at(seq * per), values: self.bufs[3].at(seq * per * self.head_dim),
                         capacity: self.capacity as i32 }
    }

    /// n_cached of sequence `seq` (kv_cache.rs:358 advances it per token).
    pub fn len(&self, seq: usize) -> usize { self.lengths[seq] as usize }

    /// prefill's attention (kv_cache.rs:121-193): normed [T][n_embd] of one
    /// prompt into slot `seq`; returns the attention output after out_proj.
    pub fn prefill(&mut self, w: &HipWaveLayer, seq: usize, normed: &[Vec<f32>]) -> Vec<Vec<f32>> {
        assert!(normed.len() <= self.capacity, "prompt longer than the cache");
        let shape = w.shape(1, normed.len());
        let kv = self.slot(seq);
        let (x, out) = (DeviceBuf::from_rows(normed), DeviceBuf::zeros(normed.len() * w.n_embd()));
        ffi::check(unsafe { ffi::wha_wave_kv_prefill(x.ptr(), &w.c(), &shape, &kv, out.ptr_mut(),
                                                     std::ptr::null_mut(), 0, std::ptr::null_mut()) },
                   "prefill");
        self.lengths[seq] = normed.len() as i32;
        out.to_rows(w.n_embd())
    }

    /// forward_one's attention (kv_cache.rs:263-335) for one new token of every
    /// sequence of the batch (normed [B][n_embd]); appends each new position.
    pub fn forward_one(&mut self, w: &HipWaveLayer, normed: &[Vec<f32>]) -> Vec<Vec<f32>> {
        assert_eq!(normed.len(), self.lengths.len());
        let shape = w.shape(normed.len(), 1);
        let kv = self.slot(0);
        let (x, out) = (DeviceBuf::from_rows(normed), DeviceBuf::zeros(normed.len() * w.n_embd()));
        ffi::check(unsafe { ffi::wha_wave_kv_decode(x.ptr(), &w.c(), &shape, &kv, self.lengths.as_ptr(),
                                                    out.ptr_mut(), std::ptr::null_mut(), 0,
                                                    std::ptr::null_mut()) }, "forward_one");
        for n in &mut self.lengths {
            *n += 1; // cache.n_cached += 1 (kv_cache.rs:358)
        }
        out.to_rows(w.n_embd())
    }
}

//! Caller-owned device buffers for the device-resident entry points (the KV
//! cache, kept scores, workspaces).  The reference owns its GPU buffers through
//! wgpu (src/wgpu_tier/ops_forward.rs:16-32); here they are plain HIP
//! allocations, freed on drop.
use std::os::raw::{c_int, c_void};

const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

extern "C" {
    fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> c_int;
    fn hipFree(ptr: *mut c_void) -> c_int;
    fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> c_int;
    fn hipMemset(dst: *mut c_void, value: c_int, size: usize) -> c_int;
    fn hipDeviceSynchronize() -> c_int;
}

fn hip_check(rc: c_int, what: &str) {
    if rc != 0 {
        panic!("{what} failed with HIP error {rc}");
    }
}

/// `len` f32 elements of device memory (hipMalloc returns 256-byte-aligned
/// blocks, which satisfies every 16-byte alignment rule of the C ABI).
pub struct DeviceBuf {
    ptr: *mut c_void,
    len: usize,
}

unsafe impl Send for DeviceBuf {}
unsafe impl Sync for DeviceBuf {}

impl DeviceBuf {
    pub fn zeros(len: usize) -> Self {
        let mut ptr = std::ptr::null_mut();
        let bytes = len.max(1) * 4;
        hip_check(unsafe { hipMalloc(&mut ptr, bytes) }, "hipMalloc");
        hip_check(unsafe { hipMemset(ptr, 0, bytes) }, "hipMemset");
        DeviceBuf { ptr, len }
    }
    pub fn from_slice(data: &[f32]) -> Self {
        let b = DeviceBuf::zeros(data.len());
        hip_check(unsafe { hipMemcpy(b.ptr, data.as_ptr() as *const c_void, data.len() * 4,
                                     HIP_MEMCPY_HOST_TO_DEVICE) }, "hipMemcpy H2D");
        b
    }
    pub fn from_rows(rows: &[Vec<f32>]) -> Self { DeviceBuf::from_slice(&rows.concat()) }
    pub fn len(&self) -> usize { self.len }
    pub fn ptr(&self) -> *const f32 { self.ptr as *const f32 }
    pub fn ptr_mut(&self) -> *mut f32 { self.ptr as *mut f32 }
    pub fn ptr_i32(&self) -> *mut i32 { self.ptr as *mut i32 }
    /// Offset view (in elements) for per-sequence slices of a batched buffer.
    pub fn at(&self, offset: usize) -> *mut f32 {
        assert!(offset <= self.len);
        unsafe { (self.ptr as *mut f32).add(offset) }
    }
    /// Waits for the device, then copies the buffer back.
    pub fn to_vec(&self) -> Vec<f32> {
        let mut out = vec![0.0f32; self.len];
        hip_check(unsafe { hipDeviceSynchronize() }, "hipDeviceSynchronize");
        hip_check(unsafe { hipMemcpy(out.as_mut_ptr() as *mut c_void, self.ptr, self.len * 4,
                                     HIP_MEMCPY_DEVICE_TO_HOST) }, "hipMemcpy D2H");
        out
    }
    pub fn to_rows(&self, width: usize) -> Vec<Vec<f32>> {
        self.to_vec().chunks(width).map(|r| r.to_vec()).collect()
    }
}

impl Drop for DeviceBuf {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            unsafe { hipFree(self.ptr) };
        }
    }
}

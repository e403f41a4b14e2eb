//! The few HIP runtime calls the safe layer needs to hold device buffers
//! (libamdhip64): allocation, copies, stream waits.  The paged-KV work itself
//! goes through liblnskv (`sys`).

use std::marker::PhantomData;
use std::mem::size_of;
use std::os::raw::{c_char, c_int, c_void};
use std::ptr;

use crate::sys::HipStream;

pub type HipError = c_int;
pub const HIP_SUCCESS: HipError = 0;
/// `hipMemcpyKind`.
pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

extern "C" {
    pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> HipError;
    pub fn hipFree(ptr: *mut c_void) -> HipError;
    pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> HipError;
    pub fn hipMemcpyAsync(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int, stream: HipStream)
        -> HipError;
    pub fn hipMemset(dst: *mut c_void, value: c_int, size: usize) -> HipError;
    pub fn hipStreamSynchronize(stream: HipStream) -> HipError;
    pub fn hipGetErrorString(err: HipError) -> *const c_char;
}

fn hip(e: HipError, what: &str) -> Result<(), String> {
    if e == HIP_SUCCESS {
        return Ok(());
    }
    let msg = unsafe { std::ffi::CStr::from_ptr(hipGetErrorString(e)) };
    Err(format!("{what}: {}", msg.to_string_lossy()))
}

/// A device array of `len` elements of a plain type, freed on drop.
pub struct DeviceBuffer<T: Copy> {
    ptr: *mut T,
    len: usize,
    _t: PhantomData<T>,
}

unsafe impl<T: Copy + Send> Send for DeviceBuffer<T> {}

impl<T: Copy> DeviceBuffer<T> {
    /// Uninitialised device memory for `len` elements.
    pub fn new(len: usize) -> Result<Self, String> {
        let mut p: *mut c_void = ptr::null_mut();
        if len > 0 {
            hip(unsafe { hipMalloc(&mut p, len * size_of::<T>()) }, "hipMalloc")?;
        }
        Ok(Self { ptr: p as *mut T, len, _t: PhantomData })
    }

    /// Device memory for `len` elements, every byte zero (decode workspaces
    /// must start so).
    pub fn zeroed(len: usize) -> Result<Self, String> {
        let b = Self::new(len)?;
        if len > 0 {
            hip(unsafe { hipMemset(b.ptr as *mut c_void, 0, len * size_of::<T>()) }, "hipMemset")?;
        }
        Ok(b)
    }

    pub fn from_slice(host: &[T]) -> Result<Self, String> {
        let mut b = Self::new(host.len())?;
        b.copy_from(host)?;
        Ok(b)
    }

    /// Host-to-device copy of `host` into the first `host.len()` elements;
    /// returns when the data is on the device (the reference writes its
    /// shared buffers from the host before committing, `engine.rs:3218-3220`).
    /// `host` into the buffer's first elements, ordered on `stream` after the
    /// work already queued there.  The runtime stages pageable host memory
    /// before the call returns, so `host` may change as soon as it does.
    pub fn copy_from_async(&mut self, host: &[T], stream: HipStream) -> Result<(), String> {
        if host.len() > self.len {
            return Err(format!("{} elements into a buffer of {}", host.len(), self.len));
        }
        if host.is_empty() {
            return Ok(());
        }
        hip(
            unsafe {
                hipMemcpyAsync(
                    self.ptr as *mut c_void,
                    host.as_ptr() as *const c_void,
                    host.len() * size_of::<T>(),
                    HIP_MEMCPY_HOST_TO_DEVICE,
                    stream,
                )
            },
            "hipMemcpyAsync host to device",
        )
    }

    pub fn copy_from(&mut self, host: &[T]) -> Result<(), String> {
        if host.len() > self.len {
            return Err(format!("{} elements into a buffer of {}", host.len(), self.len));
        }
        if host.is_empty() {
            return Ok(());
        }
        hip(
            unsafe {
                hipMemcpy(
                    self.ptr as *mut c_void,
                    host.as_ptr() as *const c_void,
                    host.len() * size_of::<T>(),
                    HIP_MEMCPY_HOST_TO_DEVICE,
                )
            },
            "hipMemcpy host to device",
        )
    }

    /// The whole buffer back to the host (waits for the null stream's work).
    pub fn to_vec(&self) -> Result<Vec<T>, String> {
        let mut v: Vec<T> = Vec::with_capacity(self.len);
        if self.len > 0 {
            hip(
                unsafe {
                    hipMemcpy(
                        v.as_mut_ptr() as *mut c_void,
                        self.ptr as *const c_void,
                        self.len * size_of::<T>(),
                        HIP_MEMCPY_DEVICE_TO_HOST,
                    )
                },
                "hipMemcpy device to host",
            )?;
            unsafe { v.set_len(self.len) };
        }
        Ok(v)
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }

    pub fn as_ptr(&self) -> *const T {
        self.ptr
    }

    pub fn as_mut_ptr(&mut self) -> *mut T {
        self.ptr
    }
}

impl<T: Copy> Drop for DeviceBuffer<T> {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            unsafe {
                let _ = hipFree(self.ptr as *mut c_void);
            }
        }
    }
}

/// Wait for the work queued on `stream`.
pub fn stream_synchronize(stream: HipStream) -> Result<(), String> {
    hip(unsafe { hipStreamSynchronize(stream) }, "hipStreamSynchronize")
}

//! `bare-metal-kernels-hip`: the public surface of RunIT's `crates/kernels`
//! (`MetalContext`, buffers, `dispatch::*`, `KernelError`) implemented over the
//! C ABI of the MI355X library (`include/runit_hip.h`, `librunit_hip.so`).
//!
//! The engine (`crates/engine/src/forward.rs`) compiles against this crate in
//! place of the Metal one: the dispatch functions keep their names and
//! argument order (`src/dispatch.rs`, generated from the header by
//! `gen_bindings.py`), `MetalContext` becomes `HipContext` with the same
//! `new` / `new_buffer` / `flush`, and `metal::Buffer` becomes [`Buffer`], a
//! device allocation that the caller owns and dispatch borrows.
//!
//! Differences that the MI355X memory model imposes (documented in
//! INTEGRATION.md): device memory is not host-visible, so host data moves
//! with [`Buffer::write`] / [`Buffer::read`] instead of `contents()`.
pub mod dispatch;
pub mod ffi;

use std::ffi::{CStr, CString};
use std::os::raw::{c_int, c_void};
use std::rc::Rc;
use thiserror::Error;

/// crates/kernels/src/error.rs:4-21, variant for variant.
#[derive(Error, Debug)]
pub enum KernelError {
    #[error("HIP device not found")]
    NoDevice,
    #[error("failed to load code object from '{path}': {reason}")]
    LibraryLoad { path: String, reason: String },
    #[error("pipeline function '{0}' not found in code object")]
    PipelineNotFound(String),
    #[error("failed to create compute pipeline for '{name}': {reason}")]
    PipelineCreate { name: String, reason: String },
    #[error("kernel dispatch error: {0}")]
    Dispatch(String),
    #[error("buffer size mismatch: expected {expected} bytes, got {actual}")]
    BufferSize { expected: usize, actual: usize },
}

pub type Result<T> = std::result::Result<T, KernelError>;

fn last_error(ctx: *const ffi::RtCtx) -> String {
    unsafe {
        let p = if ctx.is_null() { ffi::rt_global_last_error() } else { ffi::rt_last_error(ctx) };
        if p.is_null() { String::new() } else { CStr::from_ptr(p).to_string_lossy().into_owned() }
    }
}

/// The status codes of runit_hip.h (rt_status) as KernelError.
pub(crate) fn status(ctx: *const ffi::RtCtx, st: c_int) -> Result<()> {
    status_at(ctx, st, "")
}

fn status_at(ctx: *const ffi::RtCtx, st: c_int, path: &str) -> Result<()> {
    match st {
        0 => Ok(()),
        1 => Err(KernelError::NoDevice),
        2 => Err(KernelError::LibraryLoad { path: path.to_string(), reason: last_error(ctx) }),
        3 => Err(KernelError::PipelineNotFound(last_error(ctx))),
        4 => Err(KernelError::PipelineCreate { name: String::new(), reason: last_error(ctx) }),
        // the library never returns BufferSize (it validates shapes as
        // Dispatch errors); the variant is kept for the engine's own checks
        6 => Err(KernelError::BufferSize { expected: 0, actual: 0 }),
        _ => Err(KernelError::Dispatch(last_error(ctx))),
    }
}

/// `MetalContext` analogue (crates/kernels/src/context.rs:150-304): device 0,
/// the gfx950 code objects, every kernel resolved up front, one stream.
/// Not `Sync`, like `MetalContext` (context.rs:158).
///
/// The native context is reference-counted: every [`Buffer`] and [`Graph`]
/// holds a count, so the context is destroyed only when the `HipContext` and
/// everything allocated from it are gone (dropping the `HipContext` first is
/// safe; its buffers stay usable for read / write / free).
pub struct HipContext {
    inner: Rc<CtxHandle>,
    raw: *mut ffi::RtCtx,
}

/// Owner of the native context: destroyed with the last reference.
struct CtxHandle(*mut ffi::RtCtx);

impl Drop for CtxHandle {
    /// context.rs:299-304: flushes, then releases everything.
    fn drop(&mut self) {
        unsafe { ffi::rt_ctx_destroy(self.0) }
    }
}

impl HipContext {
    /// context.rs:163-205: the default code objects next to librunit_hip.so.
    pub fn new() -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        status_at(std::ptr::null(), unsafe { ffi::rt_ctx_create(&mut raw, std::ptr::null()) },
                  "<librunit_hip.so dir>/kernels")?;
        Ok(Self { inner: Rc::new(CtxHandle(raw)), raw })
    }
    /// The same with a given code object (a file, or a directory of them).
    pub fn with_code_object(path: &str) -> Result<Self> {
        let c = CString::new(path).map_err(|e| KernelError::Dispatch(e.to_string()))?;
        let mut raw = std::ptr::null_mut();
        status_at(std::ptr::null(), unsafe { ffi::rt_ctx_create(&mut raw, c.as_ptr()) }, path)?;
        Ok(Self { inner: Rc::new(CtxHandle(raw)), raw })
    }
    pub(crate) fn raw(&self) -> *mut ffi::RtCtx {
        self.raw
    }
    /// context.rs:215-220.  Device memory (zero-initialised is not promised).
    pub fn new_buffer(&self, size: usize) -> Result<Buffer> {
        let mut p = std::ptr::null_mut();
        status(self.raw, unsafe { ffi::rt_malloc(self.raw, size.max(1), &mut p) })?;
        Ok(Buffer { ptr: p, len: size, ctx: self.raw, _owner: Rc::clone(&self.inner) })
    }
    /// A new buffer holding `data` (the engine's `new_buffer` + `contents()` copy).
    pub fn buffer_from<T: Copy>(&self, data: &[T]) -> Result<Buffer> {
        let b = self.new_buffer(std::mem::size_of_val(data))?;
        b.write(data)?;
        Ok(b)
    }
    /// context.rs:289-296: waits for everything enqueued.
    pub fn flush(&self) -> Result<()> {
        status(self.raw, unsafe { ffi::rt_flush(self.raw) })
    }
    /// Records the following calls into a HIP graph instead of running them.
    pub fn capture_begin(&self) -> Result<()> {
        status(self.raw, unsafe { ffi::rt_capture_begin(self.raw) })
    }
    pub fn capture_end(&self) -> Result<Graph> {
        let mut g = std::ptr::null_mut();
        status(self.raw, unsafe { ffi::rt_capture_end(self.raw, &mut g) })?;
        Ok(Graph { raw: g, ctx: self.raw, _owner: Rc::clone(&self.inner) })
    }
}

/// A device allocation (replaces `metal::Buffer`).  The caller owns it;
/// dispatch functions borrow it.
pub struct Buffer {
    ptr: *mut c_void,
    len: usize,
    ctx: *mut ffi::RtCtx,
    _owner: Rc<CtxHandle>, // keeps the context alive until this buffer is freed
}

impl Buffer {
    pub fn as_ptr(&self) -> *mut c_void {
        self.ptr
    }
    pub fn len(&self) -> usize {
        self.len
    }
    pub fn is_empty(&self) -> bool {
        self.len == 0
    }
    /// Host → device copy of `data` at the start of the buffer (synchronous).
    pub fn write<T: Copy>(&self, data: &[T]) -> Result<()> {
        let n = std::mem::size_of_val(data);
        if n > self.len {
            return Err(KernelError::BufferSize { expected: n, actual: self.len });
        }
        status(self.ctx, unsafe { ffi::rt_upload(self.ctx, self.ptr, data.as_ptr() as *const c_void, n) })
    }
    /// Device → host copy into `out` (synchronous; waits for earlier work).
    pub fn read<T: Copy>(&self, out: &mut [T]) -> Result<()> {
        let n = std::mem::size_of_val(out);
        if n > self.len {
            return Err(KernelError::BufferSize { expected: n, actual: self.len });
        }
        status(self.ctx, unsafe { ffi::rt_download(self.ctx, out.as_mut_ptr() as *mut c_void, self.ptr, n) })
    }
}

impl Drop for Buffer {
    fn drop(&mut self) {
        unsafe { ffi::rt_free(self.ctx, self.ptr) };
    }
}

/// A captured sequence of calls (one decode step), replayed with `launch`.
pub struct Graph {
    raw: *mut ffi::RtGraph,
    ctx: *mut ffi::RtCtx,
    _owner: Rc<CtxHandle>, // keeps the context alive until the graph is destroyed
}

impl Graph {
    pub fn launch(&self) -> Result<()> {
        status(self.ctx, unsafe { ffi::rt_graph_launch(self.ctx, self.raw) })
    }
}

impl Drop for Graph {
    fn drop(&mut self) {
        unsafe { ffi::rt_graph_destroy(self.raw) }
    }
}

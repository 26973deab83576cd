//! Drop-in for foundry-spike's `AttnBwd` custom op
//! (crates/foundry-spike/src/lib.rs:151-264) that runs the MI355X (gfx950)
//! kernels of libfoundry_attn.so through its C ABI (include/foundry_attn.h).
//!
//! Same surface as the reference: a unit struct named `AttnBwd`, used as
//! `q.apply_op3(&k, &v, AttnBwd)` (lib.rs:366, 443-444; throughput.rs:548,
//! 618-619; attn_backward.rs:208-210), `name()` = "foundry-attn-bwd",
//! (S, H, D) inputs, softmax scale 1/sqrt(D) (the reference hard-codes
//! 1/sqrt(128), lib.rs:138, for its D = 128), and a `bwd` that returns
//! (dQ, dK, dV).
//!
//! Candle 0.11 has no HIP device, so the op takes the `cpu_fwd` route: like
//! the reference (lib.rs:167-172) it accepts only contiguous offset-0 inputs,
//! stages them through device buffers, runs the kernels and copies the results
//! back.  A Candle build with a HIP backend would pass its device pointers and
//! `Layout` strides (as `fa_strides`) straight through instead.
//!
//! The forward also yields each row's log-sum-exp, which lets the backward
//! recompute P without the softmax statistics.  Candle keeps only the op's
//! output, so the forward stores the LSE in a small process-wide slot keyed on
//! the addresses and shape of its q, k, v and output; `bwd` takes it from
//! there (releasing the slot's lock before any other work), and when it is not
//! there -- a different op instance, an evicted entry, a direct call -- runs
//! the forward kernel again on the same inputs into buffers the call owns,
//! which gives the same LSE bit for bit.  The reference instead recomputes
//! P in every backward (lib.rs:232-239).

mod block;
mod ffi;

pub use block::LnMod;

use candle_core::{bail, CpuStorage, CustomOp3, DType, Layout, Result, Shape, Storage, Tensor};
use std::ffi::{c_void, CStr};
use std::sync::Mutex;

/// The reference op's name (lib.rs:154-156), also what `fa_op_name` returns.
pub const OP_NAME: &str = "foundry-attn-bwd";

pub(crate) fn hip(e: ffi::hipError_t, what: &str) -> Result<()> {
    if e == ffi::HIP_SUCCESS {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(ffi::hipGetErrorString(e)) }.to_string_lossy().into_owned();
    bail!("{OP_NAME}: {what} failed: HIP error {e} ({msg})")
}

pub(crate) fn check(st: ffi::fa_status, what: &str) -> Result<()> {
    if st == ffi::FA_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(ffi::fa_last_error()) }.to_string_lossy().into_owned();
    bail!("{OP_NAME}: {what} returned status {st}: {msg}")
}

/// ABI version of the loaded library (`FA_ABI_VERSION` = 2 for these structs).
pub fn abi_version() -> i32 {
    unsafe { ffi::fa_version() }
}

/// A device buffer owned by one call, freed on drop.
pub(crate) struct DevBuf {
    pub(crate) ptr: *mut c_void,
    pub(crate) bytes: usize,
}

impl DevBuf {
    pub(crate) fn new(bytes: usize) -> Result<Self> {
        let bytes = bytes.max(256);
        let mut ptr = std::ptr::null_mut();
        hip(unsafe { ffi::hipMalloc(&mut ptr, bytes) }, "hipMalloc")?;
        Ok(Self { ptr, bytes })
    }

    pub(crate) fn upload<T: Copy>(src: &[T]) -> Result<Self> {
        let bytes = std::mem::size_of_val(src);
        let d = Self::new(bytes)?;
        if bytes > 0 {
            hip(
                unsafe {
                    ffi::hipMemcpy(d.ptr, src.as_ptr().cast(), bytes, ffi::HIP_MEMCPY_HOST_TO_DEVICE)
                },
                "hipMemcpy (host to device)",
            )?;
        }
        Ok(d)
    }

    pub(crate) fn download<T: Copy + Default>(&self, n: usize) -> Result<Vec<T>> {
        let bytes = n * std::mem::size_of::<T>();
        if bytes > self.bytes {
            bail!("{OP_NAME}: download of {bytes} bytes from a {}-byte buffer", self.bytes)
        }
        let mut v = vec![T::default(); n];
        if bytes > 0 {
            hip(
                unsafe {
                    ffi::hipMemcpy(v.as_mut_ptr().cast(), self.ptr, bytes, ffi::HIP_MEMCPY_DEVICE_TO_HOST)
                },
                "hipMemcpy (device to host)",
            )?;
        }
        Ok(v)
    }
}

impl Drop for DevBuf {
    fn drop(&mut self) {
        // Drop cannot return an error.  Every buffer is dropped after the
        // call's hipDeviceSynchronize was checked, so a failing hipFree means
        // a device error that the next checked HIP call reports.
        let _ = unsafe { ffi::hipFree(self.ptr) };
    }
}

pub(crate) fn sync() -> Result<()> {
    hip(unsafe { ffi::hipDeviceSynchronize() }, "hipDeviceSynchronize")
}

/// Dense (S, H, D) strides as the ABI's [B = 1, S, H, D] view.
fn dense(s: usize, h: usize, d: usize) -> ffi::fa_strides {
    ffi::fa_strides { b: (s * h * d) as i64, s: (h * d) as i64, h: d as i64 }
}

fn dims3(l: &Layout) -> Result<(usize, usize, usize)> {
    match l.shape().dims() {
        &[s, h, d] => Ok((s, h, d)),
        _ => bail!("{OP_NAME}: expected (seq, heads, head_dim) inputs, got {:?}", l.shape()),
    }
}

/// The reference's cpu_fwd guard (lib.rs:167-172).
pub(crate) fn require_dense(l: &Layout) -> Result<()> {
    match l.contiguous_offsets() {
        Some((0, n)) if n == l.shape().elem_count() => Ok(()),
        _ => bail!("cpu_fwd requires contiguous offset-0 inputs"),
    }
}

pub(crate) fn fa_dtype(dt: DType) -> Result<i32> {
    match dt {
        DType::F32 => Ok(ffi::FA_DTYPE_F32),
        DType::BF16 => Ok(ffi::FA_DTYPE_BF16),
        other => bail!("{OP_NAME}: dtype {other:?} is not supported (f32 or bf16)"),
    }
}

pub(crate) fn elt_bytes(dtype: i32) -> usize {
    if dtype == ffi::FA_DTYPE_F32 {
        4
    } else {
        2
    }
}

/// Address and fa_dtype of a CPU storage's data.
fn storage_ptr(s: &CpuStorage) -> Result<(usize, i32)> {
    match s {
        CpuStorage::F32(v) => Ok((v.as_ptr() as usize, ffi::FA_DTYPE_F32)),
        CpuStorage::BF16(v) => Ok((v.as_ptr() as usize, ffi::FA_DTYPE_BF16)),
        _ => bail!("{OP_NAME}: q, k and v must be f32 or bf16"),
    }
}

fn upload_storage(s: &CpuStorage) -> Result<DevBuf> {
    match s {
        CpuStorage::F32(v) => DevBuf::upload(v),
        CpuStorage::BF16(v) => DevBuf::upload(v),
        _ => bail!("{OP_NAME}: q, k and v must be f32 or bf16"),
    }
}

/// Address of a CPU tensor's first element (the key of the saved LSE).
fn tensor_ptr(t: &Tensor) -> Result<usize> {
    let (st, l) = t.storage_and_layout();
    match &*st {
        Storage::Cpu(CpuStorage::F32(v)) => Ok(v.as_ptr() as usize + 4 * l.start_offset()),
        Storage::Cpu(CpuStorage::BF16(v)) => Ok(v.as_ptr() as usize + 2 * l.start_offset()),
        _ => bail!("{OP_NAME}: bwd expects the f32 or bf16 CPU tensors of the forward"),
    }
}

// ----- the forward's LSE, kept for the backward ------------------------------

#[derive(Clone, Copy, PartialEq, Eq, Debug)]
struct LseKey {
    q: usize,
    k: usize,
    v: usize,
    out: usize,
    s: usize,
    h: usize,
    d: usize,
    dtype: i32,
}

struct SavedLse {
    key: LseKey,
    lse: Vec<f32>,
}

/// Forwards whose backward never runs (inference) must not grow this without
/// bound: the oldest entries go first.
const MAX_SAVED: usize = 16;
static SAVED: Mutex<Vec<SavedLse>> = Mutex::new(Vec::new());

fn save_lse(key: LseKey, lse: Vec<f32>) {
    let mut slot = SAVED.lock().unwrap_or_else(|p| p.into_inner());
    slot.retain(|e| e.key != key);
    if slot.len() >= MAX_SAVED {
        slot.remove(0);
    }
    slot.push(SavedLse { key, lse });
}

/// Removes and returns the LSE saved under `key`; the lock is released when
/// this returns, before the caller does anything else.
fn take_lse(key: &LseKey) -> Option<Vec<f32>> {
    let mut slot = SAVED.lock().unwrap_or_else(|p| p.into_inner());
    let i = slot.iter().position(|e| e.key == *key)?;
    Some(slot.remove(i).lse)
}

/// Runs fa_attn_fwd on device buffers; `keep` receives the workspace (if the
/// shape splits) so it outlives the asynchronous launch.
#[allow(clippy::too_many_arguments)]
fn launch_fwd(
    dtype: i32,
    (s, h, d): (usize, usize, usize),
    q: &DevBuf,
    k: &DevBuf,
    v: &DevBuf,
    o: &DevBuf,
    lse: &DevBuf,
    keep: &mut Vec<DevBuf>,
) -> Result<()> {
    let st = dense(s, h, d);
    let mut args = ffi::fa_attn_fwd_args {
        dtype,
        batch: 1,
        seq: s as i32,
        heads: h as i32,
        head_dim: d as i32,
        scale: 1.0 / (d as f32).sqrt(),
        q: q.ptr,
        k: k.ptr,
        v: v.ptr,
        o: o.ptr,
        lse: lse.ptr.cast(),
        key_keep: std::ptr::null(),
        q_stride: st,
        k_stride: st,
        v_stride: st,
        o_stride: st,
        workspace: std::ptr::null_mut(),
        workspace_bytes: 0,
    };
    // a grid too small for the GPU (few heads) splits each tile's keys when
    // given the workspace the library asks for
    let need = unsafe { ffi::fa_attn_fwd_workspace_size(&args) };
    if need > 0 {
        let ws = DevBuf::new(need)?;
        args.workspace = ws.ptr;
        args.workspace_bytes = ws.bytes;
        keep.push(ws);
    }
    check(unsafe { ffi::fa_attn_fwd(&args, std::ptr::null_mut()) }, "fa_attn_fwd")
}

/// foundry-spike's `AttnBwd` (lib.rs:151-264) on the gfx950 kernels.
#[derive(Clone, Copy, Debug, Default)]
pub struct AttnBwd;

impl CustomOp3 for AttnBwd {
    fn name(&self) -> &'static str {
        OP_NAME
    }

    fn cpu_fwd(
        &self,
        s_q: &CpuStorage,
        l_q: &Layout,
        s_k: &CpuStorage,
        l_k: &Layout,
        s_v: &CpuStorage,
        l_v: &Layout,
    ) -> Result<(CpuStorage, Shape)> {
        for l in [l_q, l_k, l_v] {
            require_dense(l)?;
        }
        let (s, h, d) = dims3(l_q)?;
        if l_k.shape() != l_q.shape() || l_v.shape() != l_q.shape() {
            bail!("{OP_NAME}: q, k and v shapes differ")
        }
        let (qp, dtype) = storage_ptr(s_q)?;
        let (kp, kdt) = storage_ptr(s_k)?;
        let (vp, vdt) = storage_ptr(s_v)?;
        if kdt != dtype || vdt != dtype {
            bail!("{OP_NAME}: q, k and v must share one dtype")
        }
        let n = s * h * d;
        let (q, k, v) = (upload_storage(s_q)?, upload_storage(s_k)?, upload_storage(s_v)?);
        let o = DevBuf::new(n * elt_bytes(dtype))?;
        let lse = DevBuf::new(h * s * 4)?;
        let mut keep = Vec::new();
        launch_fwd(dtype, (s, h, d), &q, &k, &v, &o, &lse, &mut keep)?;
        sync()?;
        let out = if dtype == ffi::FA_DTYPE_F32 {
            CpuStorage::F32(o.download::<f32>(n)?)
        } else {
            CpuStorage::BF16(o.download::<half::bf16>(n)?)
        };
        let (out_ptr, _) = storage_ptr(&out)?;
        let key = LseKey { q: qp, k: kp, v: vp, out: out_ptr, s, h, d, dtype };
        save_lse(key, lse.download::<f32>(h * s)?);
        Ok((out, l_q.shape().clone()))
    }

    fn bwd(
        &self,
        q: &Tensor,
        k: &Tensor,
        v: &Tensor,
        res: &Tensor,
        grad_res: &Tensor,
    ) -> Result<(Option<Tensor>, Option<Tensor>, Option<Tensor>)> {
        let (s, h, d) = q.dims3()?;
        for (name, t) in [("k", k), ("v", v), ("res", res), ("grad_res", grad_res)] {
            if t.dims() != q.dims() {
                bail!("{OP_NAME}: {name} shape {:?} differs from q {:?}", t.dims(), q.dims())
            }
            if t.dtype() != q.dtype() {
                bail!("{OP_NAME}: {name} dtype differs from q")
            }
        }
        let dtype = fa_dtype(q.dtype())?;
        let key = LseKey {
            q: tensor_ptr(q)?,
            k: tensor_ptr(k)?,
            v: tensor_ptr(v)?,
            out: tensor_ptr(res)?,
            s,
            h,
            d,
            dtype,
        };
        let saved = take_lse(&key);

        // every operand goes up as a dense (S, H, D) copy
        let up = |t: &Tensor| -> Result<DevBuf> {
            let t = t.contiguous()?.flatten_all()?;
            if dtype == ffi::FA_DTYPE_BF16 {
                DevBuf::upload(&t.to_vec1::<half::bf16>()?)
            } else {
                DevBuf::upload(&t.to_vec1::<f32>()?)
            }
        };
        let (qd, kd, vd, od, gd) = (up(q)?, up(k)?, up(v)?, up(res)?, up(grad_res)?);
        let n = s * h * d;
        let elt = elt_bytes(dtype);
        // buffers the launches below read or write: freed only after the sync
        let mut keep = Vec::new();
        let lse = match saved {
            Some(l) if l.len() == h * s => DevBuf::upload(&l)?,
            _ => {
                // no saved LSE: the forward again, on the same inputs, into
                // buffers this call owns (its O is discarded)
                let lse = DevBuf::new(h * s * 4)?;
                let o_scratch = DevBuf::new(n * elt)?;
                launch_fwd(dtype, (s, h, d), &qd, &kd, &vd, &o_scratch, &lse, &mut keep)?;
                keep.push(o_scratch);
                lse
            }
        };
        let (dq, dk, dv) = (DevBuf::new(n * elt)?, DevBuf::new(n * elt)?, DevBuf::new(n * elt)?);
        let st = dense(s, h, d);
        let mut args = ffi::fa_attn_bwd_args {
            dtype,
            batch: 1,
            seq: s as i32,
            heads: h as i32,
            head_dim: d as i32,
            scale: 1.0 / (d as f32).sqrt(),
            q: qd.ptr,
            k: kd.ptr,
            v: vd.ptr,
            o: od.ptr,
            dout: gd.ptr,
            lse: lse.ptr.cast(),
            key_keep: std::ptr::null(),
            dq: dq.ptr,
            dk: dk.ptr,
            dv: dv.ptr,
            workspace: std::ptr::null_mut(),
            workspace_bytes: 0,
            q_stride: st,
            k_stride: st,
            v_stride: st,
            o_stride: st,
            do_stride: st,
            dq_stride: st,
            dk_stride: st,
            dv_stride: st,
        };
        let ws = DevBuf::new(unsafe { ffi::fa_attn_bwd_workspace_size(&args) })?;
        args.workspace = ws.ptr;
        args.workspace_bytes = ws.bytes;
        check(unsafe { ffi::fa_attn_bwd(&args, std::ptr::null_mut()) }, "fa_attn_bwd")?;
        sync()?;
        drop(keep);
        let down = |b: &DevBuf| -> Result<Tensor> {
            if dtype == ffi::FA_DTYPE_BF16 {
                Tensor::from_vec(b.download::<half::bf16>(n)?, (s, h, d), q.device())
            } else {
                Tensor::from_vec(b.download::<f32>(n)?, (s, h, d), q.device())
            }
        };
        Ok((Some(down(&dq)?), Some(down(&dk)?), Some(down(&dv)?)))
    }
}

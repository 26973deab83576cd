//! `layer_norm_mod` (crates/foundry-spike/src/lib.rs:60-71) as a Candle
//! `CustomOp3` over fa_ln_mod_fwd / fa_ln_mod_bwd (include/foundry_block.h):
//! the pattern the other block ops (fa_gated_residual, fa_swiglu_*,
//! fa_adamw_step) follow.  Same cpu_fwd route as `AttnBwd`: contiguous
//! offset-0 CPU inputs, staged through device buffers.

use crate::{check, elt_bytes, fa_dtype, ffi, require_dense, sync, DevBuf};
use candle_core::{bail, CpuStorage, CustomOp3, Layout, Result, Shape, Tensor};

/// `x.apply_op3(&shift, &scale, LnMod { eps })` where the reference calls
/// `layer_norm_mod(x, shift, scale, eps)`: LayerNorm without affine over the
/// last dimension in f32, then (1 + scale) * n + shift, cast back.  shift and
/// scale are the frozen modulation parts (`mod_parts`, throughput.rs:297-324),
/// so the backward returns a gradient for x only.
#[derive(Clone, Copy, Debug)]
pub struct LnMod {
    pub eps: f32,
}

/// (rows, cols) of x with every leading dimension folded into rows.
fn rows_cols(dims: &[usize]) -> Result<(usize, usize)> {
    match dims.split_last() {
        Some((&c, lead)) if c > 0 => Ok((lead.iter().product(), c)),
        _ => bail!("foundry-ln-mod: x needs a non-empty last dimension"),
    }
}

fn upload_storage(s: &CpuStorage) -> Result<(DevBuf, i32)> {
    match s {
        CpuStorage::F32(v) => Ok((DevBuf::upload(v)?, ffi::FA_DTYPE_F32)),
        CpuStorage::BF16(v) => Ok((DevBuf::upload(v)?, ffi::FA_DTYPE_BF16)),
        _ => bail!("foundry-ln-mod: x, shift and scale must be f32 or bf16"),
    }
}

impl CustomOp3 for LnMod {
    fn name(&self) -> &'static str {
        "foundry-ln-mod"
    }

    fn cpu_fwd(
        &self,
        sx: &CpuStorage,
        lx: &Layout,
        ssh: &CpuStorage,
        lsh: &Layout,
        ssc: &CpuStorage,
        lsc: &Layout,
    ) -> Result<(CpuStorage, Shape)> {
        for l in [lx, lsh, lsc] {
            require_dense(l)?;
        }
        let (rows, cols) = rows_cols(lx.shape().dims())?;
        if lsh.shape().elem_count() != cols || lsc.shape().elem_count() != cols {
            bail!("foundry-ln-mod: shift and scale must hold {cols} values")
        }
        let (x, dtype) = upload_storage(sx)?;
        let (sh, dt1) = upload_storage(ssh)?;
        let (sc, dt2) = upload_storage(ssc)?;
        if dt1 != dtype || dt2 != dtype {
            bail!("foundry-ln-mod: x, shift and scale must share one dtype")
        }
        let y = DevBuf::new(rows * cols * elt_bytes(dtype))?;
        let args = ffi::fa_ln_mod_args {
            dtype,
            rows: rows as i32,
            cols: cols as i32,
            eps: self.eps,
            x: x.ptr,
            ldx: cols as i64,
            shift: sh.ptr,
            scale: sc.ptr,
            y: y.ptr,
            ldy: cols as i64,
            mean: std::ptr::null_mut(),
            rstd: std::ptr::null_mut(),
        };
        check(unsafe { ffi::fa_ln_mod_fwd(&args, std::ptr::null_mut()) }, "fa_ln_mod_fwd")?;
        sync()?;
        let out = if dtype == ffi::FA_DTYPE_F32 {
            CpuStorage::F32(y.download::<f32>(rows * cols)?)
        } else {
            CpuStorage::BF16(y.download::<half::bf16>(rows * cols)?)
        };
        Ok((out, lx.shape().clone()))
    }

    fn bwd(
        &self,
        x: &Tensor,
        shift: &Tensor,
        scale: &Tensor,
        _res: &Tensor,
        dy: &Tensor,
    ) -> Result<(Option<Tensor>, Option<Tensor>, Option<Tensor>)> {
        let (rows, cols) = rows_cols(x.dims())?;
        let dtype = fa_dtype(x.dtype())?;
        if dy.dims() != x.dims() {
            bail!("foundry-ln-mod: dy shape {:?} differs from x {:?}", dy.dims(), x.dims())
        }
        let up = |t: &Tensor| -> Result<DevBuf> {
            let t = t.contiguous()?.flatten_all()?;
            if dtype == ffi::FA_DTYPE_BF16 {
                DevBuf::upload(&t.to_vec1::<half::bf16>()?)
            } else {
                DevBuf::upload(&t.to_vec1::<f32>()?)
            }
        };
        let (xd, shd, scd, dyd) = (up(x)?, up(shift)?, up(scale)?, up(dy)?);
        let elt = elt_bytes(dtype);
        // the forward again for the row statistics (mean, rstd), then the
        // backward; y is written and discarded
        let y = DevBuf::new(rows * cols * elt)?;
        let mean = DevBuf::new(rows * 4)?;
        let rstd = DevBuf::new(rows * 4)?;
        let dx = DevBuf::new(rows * cols * elt)?;
        let fwd = ffi::fa_ln_mod_args {
            dtype,
            rows: rows as i32,
            cols: cols as i32,
            eps: self.eps,
            x: xd.ptr,
            ldx: cols as i64,
            shift: shd.ptr,
            scale: scd.ptr,
            y: y.ptr,
            ldy: cols as i64,
            mean: mean.ptr.cast(),
            rstd: rstd.ptr.cast(),
        };
        check(unsafe { ffi::fa_ln_mod_fwd(&fwd, std::ptr::null_mut()) }, "fa_ln_mod_fwd")?;
        let args = ffi::fa_ln_mod_bwd_args {
            fwd,
            dy: dyd.ptr,
            lddy: cols as i64,
            dres: std::ptr::null(),
            ldres: 0,
            dx: dx.ptr,
            lddx: cols as i64,
        };
        check(unsafe { ffi::fa_ln_mod_bwd(&args, std::ptr::null_mut()) }, "fa_ln_mod_bwd")?;
        sync()?;
        let n = rows * cols;
        let t = if dtype == ffi::FA_DTYPE_BF16 {
            Tensor::from_vec(dx.download::<half::bf16>(n)?, x.dims(), x.device())?
        } else {
            Tensor::from_vec(dx.download::<f32>(n)?, x.dims(), x.device())?
        };
        Ok((Some(t), None, None))
    }
}

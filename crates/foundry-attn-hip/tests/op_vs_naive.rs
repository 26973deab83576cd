//! The op against a plain f64 restatement of the reference's attention and
//! its gradients (lib.rs:131-149, 216-263), on config c1's shape (S = 256,
//! H = 4, D = 64, f32, seeded N(0,1) inputs).  Needs a gfx950 GPU and
//! libfoundry_attn.so (FOUNDRY_ATTN_LIB_DIR at build time).
//!
//! The upstream gradient enters through the reference's seed trick
//! (attn_backward.rs:220-222): loss = sum(O * dO) makes dL/dO = dO.

use candle_core::{CustomOp3, Device, Result, Tensor, Var};
use foundry_attn_hip::{abi_version, AttnBwd, OP_NAME};

const S: usize = 256;
const H: usize = 4;
const D: usize = 64;

/// Deterministic N(0,1) values (64-bit LCG + Box-Muller).
fn normals(n: usize, seed: u64) -> Vec<f32> {
    let mut x = seed.wrapping_mul(6364136223846793005).wrapping_add(1442695040888963407);
    let mut uniform = move || {
        x = x.wrapping_mul(6364136223846793005).wrapping_add(1442695040888963407);
        ((x >> 11) as f64 + 0.5) / (1u64 << 53) as f64
    };
    (0..n)
        .map(|_| {
            let (u1, u2) = (uniform(), uniform());
            ((-2.0 * u1.ln()).sqrt() * (2.0 * std::f64::consts::PI * u2).cos()) as f32
        })
        .collect()
}

struct Naive {
    o: Vec<f64>,
    dq: Vec<f64>,
    dk: Vec<f64>,
    dv: Vec<f64>,
}

/// Materialised attention and its gradients in f64, [S, H, D] row-major.
fn naive(q: &[f32], k: &[f32], v: &[f32], g: &[f32]) -> Naive {
    let at = |t: &[f32], s: usize, h: usize, f: usize| t[(s * H + h) * D + f] as f64;
    let scale = 1.0 / (D as f64).sqrt();
    let n = S * H * D;
    let (mut o, mut dq, mut dk, mut dv) = (vec![0.0; n], vec![0.0; n], vec![0.0; n], vec![0.0; n]);
    for h in 0..H {
        for i in 0..S {
            let sc: Vec<f64> =
                (0..S).map(|j| scale * (0..D).map(|f| at(q, i, h, f) * at(k, j, h, f)).sum::<f64>()).collect();
            let m = sc.iter().cloned().fold(f64::NEG_INFINITY, f64::max);
            let e: Vec<f64> = sc.iter().map(|x| (x - m).exp()).collect();
            let z: f64 = e.iter().sum();
            let p: Vec<f64> = e.iter().map(|x| x / z).collect();
            let dp: Vec<f64> = (0..S).map(|j| (0..D).map(|f| at(g, i, h, f) * at(v, j, h, f)).sum()).collect();
            let delta: f64 = (0..S).map(|j| p[j] * dp[j]).sum();
            for j in 0..S {
                let ds = p[j] * (dp[j] - delta) * scale;
                for f in 0..D {
                    let idx = (i * H + h) * D + f;
                    let jdx = (j * H + h) * D + f;
                    o[idx] += p[j] * at(v, j, h, f);
                    dq[idx] += ds * at(k, j, h, f);
                    dk[jdx] += ds * at(q, i, h, f);
                    dv[jdx] += p[j] * at(g, i, h, f);
                }
            }
        }
    }
    Naive { o, dq, dk, dv }
}

fn rel_l2(got: &Tensor, want: &[f64]) -> Result<f64> {
    let got: Vec<f32> = got.flatten_all()?.to_vec1()?;
    let (mut num, mut den) = (0.0, 0.0);
    for (a, b) in got.iter().zip(want) {
        num += (*a as f64 - b) * (*a as f64 - b);
        den += b * b;
    }
    Ok((num / den).sqrt())
}

#[test]
fn name_and_abi() {
    assert_eq!(AttnBwd.name(), OP_NAME);
    assert_eq!(AttnBwd.name(), "foundry-attn-bwd");
    assert_eq!(abi_version(), 2);
}

#[test]
fn c1_forward_and_backward_match_naive() -> Result<()> {
    let dev = Device::Cpu;
    let (q, k, v, g) = (normals(S * H * D, 1), normals(S * H * D, 2), normals(S * H * D, 3), normals(S * H * D, 4));
    let want = naive(&q, &k, &v, &g);
    let qv = Var::from_tensor(&Tensor::from_vec(q, (S, H, D), &dev)?)?;
    let kv = Var::from_tensor(&Tensor::from_vec(k, (S, H, D), &dev)?)?;
    let vv = Var::from_tensor(&Tensor::from_vec(v, (S, H, D), &dev)?)?;
    let gt = Tensor::from_vec(g, (S, H, D), &dev)?;
    let o = qv.as_tensor().apply_op3(kv.as_tensor(), vv.as_tensor(), AttnBwd)?;
    assert!(rel_l2(&o, &want.o)? <= 1e-4, "O");
    let grads = (&o * &gt)?.sum_all()?.backward()?;
    for (name, var, w) in [("dQ", &qv, &want.dq), ("dK", &kv, &want.dk), ("dV", &vv, &want.dv)] {
        let got = grads.get(var.as_tensor()).expect("gradient");
        let r = rel_l2(got, w)?;
        assert!(r <= 1e-4, "{name} rel-L2 {r:e}");
    }
    // a direct call with no saved LSE regenerates it and gives the same bits
    let (dq2, _, _) = AttnBwd.bwd(qv.as_tensor(), kv.as_tensor(), vv.as_tensor(), &o, &gt)?;
    let a: Vec<f32> = grads.get(qv.as_tensor()).unwrap().flatten_all()?.to_vec1()?;
    let b: Vec<f32> = dq2.unwrap().flatten_all()?.to_vec1()?;
    assert_eq!(a, b);
    Ok(())
}

#[test]
fn cpu_fwd_refuses_offset_views_like_the_reference() -> Result<()> {
    let dev = Device::Cpu;
    let big = Tensor::from_vec(normals((S + 1) * H * D, 5), (S + 1, H, D), &dev)?;
    let q = big.narrow(0, 1, S)?; // offset view: lib.rs:167-172 bails on it
    let k = Tensor::from_vec(normals(S * H * D, 6), (S, H, D), &dev)?;
    let err = q.apply_op3(&k, &k, AttnBwd).unwrap_err().to_string();
    assert!(err.contains("contiguous offset-0"), "{err}");
    Ok(())
}

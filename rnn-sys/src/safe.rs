//! Safe layer of rnn-sys: the reference's GEMM-core call sites with their own
//! signatures, computed on the GPU through the `*_host` entry points of
//! librnn.so (operands copied in, one device call, outputs copied back).
//!
//! * `matmul`, `gemm_small`, `matmul_dw` keep gemm.rs:434, 500 and 555
//!   exactly: `use rnn_sys::safe::{matmul, gemm_small, matmul_dw, PackedA,
//!   PackedB};` replaces the CPU versions at every caller.
//! * `Core` keeps attn.rs:75-84's fields and the parameter lists of
//!   `Core::forward` / `Core::backward` (attn.rs:148-160, 226-242), so
//!   SelfAttn / CrossAttn (attn.rs:346-560) run unchanged on top of it.
//! * `conv2d_forward` / `conv2d_backward_w` / `conv2d_backward_x` and
//!   `linear_forward` / `linear_backward` are the bodies of
//!   `Conv2d::{forward, backward_w, backward}` (nn.rs:166, 193, 230) and
//!   `Linear::{forward, backward}` (linear.rs:44, 66) over slices: those
//!   methods keep their signatures and their bodies become one call of
//!   these.
//!
//! Errors panic, which the reference's `panic = "abort"` turns into an abort,
//! as a slice-bounds panic there does.  One library context serves the
//! process (device `RNN_DEVICE`, default 0); calls from several threads are
//! serialised on it, as the context's stream would serialise them anyway.
use crate::*;
use std::ffi::CStr;
use std::os::raw::c_int;
use std::sync::Mutex;

struct Ctx(*mut rnn_ctx);
// The context is only used under CTX's lock.
unsafe impl Send for Ctx {}

static CTX: Mutex<Option<Ctx>> = Mutex::new(None);

fn check(ctx: *mut rnn_ctx, rc: c_int, what: &str) {
    if rc == RNN_OK {
        return;
    }
    let msg = unsafe {
        let p = if ctx.is_null() { std::ptr::null() } else { rnn_ctx_last_error(ctx) };
        let p = if p.is_null() || *p == 0 { rnn_status_string(rc) } else { p };
        CStr::from_ptr(p).to_string_lossy().into_owned()
    };
    panic!("{what}: {msg} (status {rc})");
}

fn with_ctx<R>(f: impl FnOnce(*mut rnn_ctx) -> R) -> R {
    let mut g = CTX.lock().unwrap_or_else(|e| e.into_inner());
    if g.is_none() {
        let dev = std::env::var("RNN_DEVICE").ok().and_then(|s| s.parse().ok()).unwrap_or(0);
        let mut h: *mut rnn_ctx = std::ptr::null_mut();
        check(std::ptr::null_mut(), unsafe { rnn_ctx_create(dev, &mut h) }, "rnn_ctx_create");
        *g = Some(Ctx(h));
    }
    f(g.as_ref().unwrap().0)
}

fn need(len: usize, want: usize, what: &str) {
    assert!(len >= want, "{what}: slice of {len} elements, {want} needed");
}

// ------------------------------------------------------------------ gemm.rs

/// Stand-in for gemm.rs's packing buffer (gemm.rs:21-120).  The device
/// kernels stage their operands in LDS, so it holds nothing; it exists so
/// that `gemm_small`'s callers keep their scratch arguments.
#[derive(Default)]
pub struct PackedA;
impl PackedA {
    pub fn new() -> PackedA {
        PackedA
    }
}

/// Stand-in for gemm.rs's PackedB (gemm.rs:306-407); see PackedA.
#[derive(Default)]
pub struct PackedB;
impl PackedB {
    pub fn new() -> PackedB {
        PackedB
    }
}

/// matmul (gemm.rs:434-493): C[m x n] = op(A) op(B) (+ C when acc); at: A is
/// [k x m]; bt: B is [n x k].  m or n = 0: nothing; k = 0: C = 0 unless acc.
#[allow(clippy::too_many_arguments)]
pub fn matmul(
    m: usize,
    n: usize,
    k: usize,
    a: &[f32],
    at: bool,
    b: &[f32],
    bt: bool,
    c: &mut [f32],
    acc: bool,
) {
    if m == 0 || n == 0 {
        return;
    }
    need(a.len(), m * k, "matmul a");
    need(b.len(), k * n, "matmul b");
    need(c.len(), m * n, "matmul c");
    with_ctx(|ctx| {
        let rc = unsafe {
            rnn_matmul_host(ctx, m, n, k, a.as_ptr(), at as c_int, b.as_ptr(), bt as c_int,
                            c.as_mut_ptr(), acc as c_int)
        };
        check(ctx, rc, "matmul");
    })
}

/// gemm_small (gemm.rs:500-545): matmul's product for one small problem;
/// k = 0 leaves C untouched.  The packing buffers are not used.
#[allow(clippy::too_many_arguments)]
pub fn gemm_small(
    m: usize,
    n: usize,
    k: usize,
    a: &[f32],
    at: bool,
    b: &[f32],
    bt: bool,
    c: &mut [f32],
    acc: bool,
    _ap: &mut PackedA,
    _bp: &mut PackedB,
) {
    if m == 0 || n == 0 {
        return;
    }
    need(a.len(), m * k, "gemm_small a");
    need(b.len(), k * n, "gemm_small b");
    need(c.len(), m * n, "gemm_small c");
    with_ctx(|ctx| {
        let rc = unsafe {
            rnn_gemm_small_batched_host(ctx, 1, m, n, k, a.as_ptr(), m * k, at as c_int,
                                        b.as_ptr(), k * n, bt as c_int, c.as_mut_ptr(), m * n,
                                        acc as c_int)
        };
        check(ctx, rc, "gemm_small");
    })
}

/// matmul_dw (gemm.rs:547-598): C[m x n] += A^T B with A [k x m], B [k x n].
pub fn matmul_dw(m: usize, n: usize, k: usize, a: &[f32], b: &[f32], c: &mut [f32]) {
    if m == 0 || n == 0 || k == 0 {
        return;
    }
    need(a.len(), k * m, "matmul_dw a");
    need(b.len(), k * n, "matmul_dw b");
    need(c.len(), m * n, "matmul_dw c");
    with_ctx(|ctx| {
        let rc = unsafe { rnn_matmul_dw_host(ctx, m, n, k, a.as_ptr(), b.as_ptr(), c.as_mut_ptr()) };
        check(ctx, rc, "matmul_dw");
    })
}

// ------------------------------------------------------------------ conv.rs

/// ConvSpec (conv.rs:9-20) with oh / ow from Conv2d::out_dim (nn.rs:147-150).
#[derive(Clone, Copy, Debug)]
pub struct ConvSpec {
    pub cin: usize,
    pub cout: usize,
    pub k: usize,
    pub stride: usize,
    pub pad: usize,
    pub h: usize,
    pub w: usize,
    pub oh: usize,
    pub ow: usize,
}

impl ConvSpec {
    fn raw(&self) -> rnn_conv_spec {
        let u = |v: usize| u32::try_from(v).expect("conv spec field beyond u32");
        rnn_conv_spec {
            cin: u(self.cin),
            cout: u(self.cout),
            k: u(self.k),
            stride: u(self.stride),
            pad: u(self.pad),
            h: u(self.h),
            w: u(self.w),
            oh: u(self.oh),
            ow: u(self.ow),
        }
    }
    fn lens(&self, n: usize) -> (usize, usize, usize) {
        (n * self.cin * self.h * self.w, self.cout * self.cin * self.k * self.k,
         n * self.cout * self.oh * self.ow)
    }
}

/// Body of Conv2d::forward (nn.rs:166-185): y[n][cout][oh][ow] = W im2col(x)
/// for the n images of x (overwritten).
pub fn conv2d_forward(sp: &ConvSpec, n: usize, x: &[f32], w: &[f32], y: &mut [f32]) {
    let (lx, lw, ly) = sp.lens(n);
    need(x.len(), lx, "conv2d_forward x");
    need(w.len(), lw, "conv2d_forward w");
    need(y.len(), ly, "conv2d_forward y");
    let raw = sp.raw();
    with_ctx(|ctx| {
        let rc = unsafe {
            rnn_conv2d_forward_host(ctx, &raw, n, x.as_ptr(), w.as_ptr(), y.as_mut_ptr())
        };
        check(ctx, rc, "conv2d_forward");
    })
}

/// Body of Conv2d::backward_w (nn.rs:193-227): dw[cout][cin*k*k] += the sum
/// over the batch of dY im2col(X)^T (W's gradient accumulates, as w.g does).
pub fn conv2d_backward_w(sp: &ConvSpec, n: usize, dy: &[f32], x: &[f32], dw: &mut [f32]) {
    let (lx, lw, ly) = sp.lens(n);
    need(dy.len(), ly, "conv2d_backward_w dy");
    need(x.len(), lx, "conv2d_backward_w x");
    need(dw.len(), lw, "conv2d_backward_w dw");
    let raw = sp.raw();
    with_ctx(|ctx| {
        let rc = unsafe {
            rnn_conv2d_backward_w_host(ctx, &raw, n, dy.as_ptr(), x.as_ptr(), dw.as_mut_ptr())
        };
        check(ctx, rc, "conv2d_backward_w");
    })
}

/// dX half of Conv2d::backward (nn.rs:230-250): dx = col2im(W^T dY)
/// (overwritten, as the zero-filled Tensor there is).
pub fn conv2d_backward_x(sp: &ConvSpec, n: usize, dy: &[f32], w: &[f32], dx: &mut [f32]) {
    let (lx, lw, ly) = sp.lens(n);
    need(dy.len(), ly, "conv2d_backward_x dy");
    need(w.len(), lw, "conv2d_backward_x w");
    need(dx.len(), lx, "conv2d_backward_x dx");
    let raw = sp.raw();
    with_ctx(|ctx| {
        let rc = unsafe {
            rnn_conv2d_backward_x_host(ctx, &raw, n, dy.as_ptr(), w.as_ptr(), dx.as_mut_ptr())
        };
        check(ctx, rc, "conv2d_backward_x");
    })
}

// ------------------------------------------------------------------ attn.rs

/// Core (attn.rs:75-84): the parameters SelfAttn and CrossAttn share, with
/// the same fields; `relidx` / `nrel` come from rel_index (attn.rs:53-72, or
/// rnn_rel_index).
pub struct Core {
    pub h: usize,
    pub dh: usize,
    pub tq: usize,
    pub tk: usize,
    pub relidx: Vec<u32>,
    pub nrel: usize,
    pub mask_diag: bool,
}

impl Core {
    // Floats the strided query and key / value buffers of n images span
    // (row r at r*stride, the last row's heads ending at off + h*dh).
    fn extents(&self, n: usize, qstride: usize, qoff: usize, kvstride: usize, koff: usize,
               voff: usize) -> (usize, usize) {
        let hdh = self.h * self.dh;
        ((n * self.tq - 1) * qstride + qoff + hdh,
         (n * self.tk - 1) * kvstride + koff.max(voff) + hdh)
    }

    #[allow(clippy::too_many_arguments)]
    fn desc(&self, qstride: usize, qoff: usize, kvstride: usize, koff: usize,
            voff: usize) -> rnn_attn_desc {
        let u = |v: usize| u32::try_from(v).expect("attention size beyond u32");
        assert_eq!(self.relidx.len(), self.tq * self.tk, "relidx must hold tq*tk entries");
        rnn_attn_desc {
            h: u(self.h),
            dh: u(self.dh),
            tq: u(self.tq),
            tk: u(self.tk),
            qstride,
            qoff,
            kvstride,
            koff,
            voff,
            nrel: u(self.nrel),
            relidx: self.relidx.as_ptr(),
            mask_diag: self.mask_diag as c_int,
        }
    }

    /// Core::forward (attn.rs:148-223): per image and head s = tau QK^T +
    /// rel (diagonal masked when mask_diag), p = softmax(s), o = p V; the
    /// batch is o.len() / (tq h dh) images.
    #[allow(clippy::too_many_arguments)]
    pub fn forward(
        &self,
        q: &[f32],
        qstride: usize,
        qoff: usize,
        kv: &[f32],
        kvstride: usize,
        koff: usize,
        voff: usize,
        tau: &[f32],
        rel: &[f32],
        p: &mut [f32],
        o: &mut [f32],
    ) {
        let c = self.h * self.dh;
        let n = o.len() / (self.tq * c);
        if n == 0 {
            return;
        }
        let (nq, nkv) = self.extents(n, qstride, qoff, kvstride, koff, voff);
        need(q.len(), nq, "Core::forward q");
        need(kv.len(), nkv, "Core::forward kv");
        need(tau.len(), self.h, "Core::forward tau");
        need(rel.len(), self.h * self.nrel, "Core::forward rel");
        need(p.len(), n * self.h * self.tq * self.tk, "Core::forward p");
        let d = self.desc(qstride, qoff, kvstride, koff, voff);
        with_ctx(|ctx| {
            let rc = unsafe {
                rnn_attn_forward_host(ctx, &d, n, q.as_ptr(), kv.as_ptr(), tau.as_ptr(),
                                      rel.as_ptr(), p.as_mut_ptr(), o.as_mut_ptr())
            };
            check(ctx, rc, "Core::forward");
        })
    }

    /// Core::backward (attn.rs:226-343): dq, dkv, dtau and drel accumulate.
    /// dq and dkv are distinct buffers here (SelfAttn::backward passes two
    /// zeroed ones and adds them afterwards, attn.rs:418-438); the C entry
    /// point also accepts one buffer for both.
    #[allow(clippy::too_many_arguments)]
    pub fn backward(
        &self,
        q: &[f32],
        qstride: usize,
        qoff: usize,
        kv: &[f32],
        kvstride: usize,
        koff: usize,
        voff: usize,
        tau: &[f32],
        p: &[f32],
        dobuf: &[f32],
        dq: &mut [f32],
        dkv: &mut [f32],
        dtau: &mut [f32],
        drel: &mut [f32],
    ) {
        let c = self.h * self.dh;
        let n = dobuf.len() / (self.tq * c);
        if n == 0 {
            return;
        }
        let (nq, nkv) = self.extents(n, qstride, qoff, kvstride, koff, voff);
        need(q.len(), nq, "Core::backward q");
        need(kv.len(), nkv, "Core::backward kv");
        need(tau.len(), self.h, "Core::backward tau");
        need(p.len(), n * self.h * self.tq * self.tk, "Core::backward p");
        need(dq.len(), nq, "Core::backward dq");
        need(dkv.len(), nkv, "Core::backward dkv");
        need(dtau.len(), self.h, "Core::backward dtau");
        need(drel.len(), self.h * self.nrel, "Core::backward drel");
        let d = self.desc(qstride, qoff, kvstride, koff, voff);
        with_ctx(|ctx| {
            let rc = unsafe {
                rnn_attn_backward_host(ctx, &d, n, q.as_ptr(), kv.as_ptr(), tau.as_ptr(),
                                       p.as_ptr(), dobuf.as_ptr(), dq.as_mut_ptr(),
                                       dkv.as_mut_ptr(), dtau.as_mut_ptr(), drel.as_mut_ptr())
            };
            check(ctx, rc, "Core::backward");
        })
    }
}

// ---------------------------------------------------------------- linear.rs

/// Body of Linear::forward (linear.rs:44-64): y[rows][fout] = x W^T + b.
pub fn linear_forward(w: &[f32], b: Option<&[f32]>, fin: usize, fout: usize, x: &[f32],
                      rows: usize) -> Vec<f32> {
    let mut y = vec![0.0f32; rows * fout];
    if rows == 0 || fout == 0 {
        return y;
    }
    need(w.len(), fout * fin, "Linear::forward w");
    need(x.len(), rows * fin, "Linear::forward x");
    if let Some(b) = b {
        need(b.len(), fout, "Linear::forward b");
    }
    with_ctx(|ctx| {
        let rc = unsafe {
            rnn_linear_forward_host(ctx, rows, fin, fout, x.as_ptr(), w.as_ptr(),
                                    b.map_or(std::ptr::null(), |b| b.as_ptr()), y.as_mut_ptr())
        };
        check(ctx, rc, "Linear::forward");
    });
    y
}

/// Body of Linear::backward (linear.rs:66-96): dw += dy^T x, db += the
/// column sums of dy, returns dx = dy W.
#[allow(clippy::too_many_arguments)]
pub fn linear_backward(w: &[f32], dw: &mut [f32], db: Option<&mut [f32]>, fin: usize,
                       fout: usize, x: &[f32], dy: &[f32], rows: usize) -> Vec<f32> {
    let mut dx = vec![0.0f32; rows * fin];
    if rows == 0 {
        return dx;
    }
    need(w.len(), fout * fin, "Linear::backward w");
    need(dw.len(), fout * fin, "Linear::backward dw");
    need(x.len(), rows * fin, "Linear::backward x");
    need(dy.len(), rows * fout, "Linear::backward dy");
    let dbp = match db {
        Some(d) => {
            need(d.len(), fout, "Linear::backward db");
            d.as_mut_ptr()
        }
        None => std::ptr::null_mut(),
    };
    with_ctx(|ctx| {
        let rc = unsafe {
            rnn_linear_backward_host(ctx, rows, fin, fout, dy.as_ptr(), x.as_ptr(), w.as_ptr(),
                                     dw.as_mut_ptr(), dbp, dx.as_mut_ptr())
        };
        check(ctx, rc, "Linear::backward");
    });
    dx
}

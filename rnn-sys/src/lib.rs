// Generated from include/rnn.h by rnn-sys/gen_bindings.py; do not edit.
// The C ABI of librnn.so (the MI355X GEMM core of rustnn).
#![allow(non_camel_case_types)]
use std::os::raw::{c_char, c_int, c_void};

pub const RNN_OK: c_int = 0;
pub const RNN_E_INVALID: c_int = -1;
pub const RNN_E_NULL: c_int = -2;
pub const RNN_E_HIP: c_int = -3;
pub const RNN_E_NOMEM: c_int = -4;
pub const RNN_E_UNSUPPORTED: c_int = -5;
pub const RNN_ATTN_SET_DQ: u32 = 1;
pub const RNN_ATTN_SET_DKV: u32 = 2;
pub const RNN_LINEAR_ACC_DX: u32 = 1;
pub const RNN_DW3_ACC_DX: u32 = 1;

#[repr(C)] pub struct rnn_ctx { _p: [u8; 0] }
#[repr(C)] pub struct rnn_conv_packs { _p: [u8; 0] }
#[repr(C)] pub struct rnn_optim { _p: [u8; 0] }
#[repr(C)] pub struct rnn_resnet { _p: [u8; 0] }

#[repr(C)] #[derive(Clone, Copy)]
pub struct rnn_conv_spec {
    pub cin: u32,
    pub cout: u32,
    pub k: u32,
    pub stride: u32,
    pub pad: u32,
    pub h: u32,
    pub w: u32,
    pub oh: u32,
    pub ow: u32,
}

#[repr(C)] #[derive(Clone, Copy)]
pub struct rnn_attn_desc {
    pub h: u32,
    pub dh: u32,
    pub tq: u32,
    pub tk: u32,
    pub qstride: usize,
    pub qoff: usize,
    pub kvstride: usize,
    pub koff: usize,
    pub voff: usize,
    pub nrel: u32,
    pub relidx: *const u32,
    pub mask_diag: c_int,
}

#[repr(C)] #[derive(Clone, Copy)]
pub struct rnn_loss_cfg {
    pub coarse_w: f32,
    pub exit_w1: f32,
    pub exit_w2: f32,
    pub alpha: f32,
    pub temp: f32,
    pub beta: f32,
    pub taxo: c_int,
}

#[repr(C)] #[derive(Clone, Copy)]
pub struct rnn_loss_io {
    pub logits: *const f32,
    pub coarse: *const f32,
    pub e1: *const f32,
    pub e2: *const f32,
    pub h1: *const f32,
    pub h2: *const f32,
    pub feat: *const f32,
    pub dlogits: *mut f32,
    pub dcoarse: *mut f32,
    pub de1: *mut f32,
    pub de2: *mut f32,
    pub dh1: *mut f32,
    pub dh2: *mut f32,
}

#[repr(C)] #[derive(Clone, Copy)]
pub struct rnn_param {
    pub v: *mut f32,
    pub g: *mut f32,
    pub m: *mut f32,
    pub v2: *mut f32,
    pub len: usize,
    pub rows: usize,
    pub cols: usize,
    pub decay: c_int,
}

#[link(name = "rnn")]
extern "C" {
    pub fn rnn_ctx_create(device: c_int, out: *mut *mut rnn_ctx) -> c_int;
    pub fn rnn_ctx_destroy(ctx: *mut rnn_ctx) -> c_int;
    pub fn rnn_ctx_set_stream(ctx: *mut rnn_ctx, stream: *mut c_void) -> c_int;
    pub fn rnn_ctx_set_defer(ctx: *mut rnn_ctx, on: c_int) -> c_int;
    pub fn rnn_ctx_flush(ctx: *mut rnn_ctx) -> c_int;
    pub fn rnn_ctx_stream(ctx: *mut rnn_ctx) -> *mut c_void;
    pub fn rnn_ctx_synchronize(ctx: *mut rnn_ctx) -> c_int;
    pub fn rnn_ctx_last_error(ctx: *mut rnn_ctx) -> *const c_char;
    pub fn rnn_status_string(status: c_int) -> *const c_char;
    pub fn rnn_ctx_workspace_bytes(ctx: *mut rnn_ctx) -> usize;
    pub fn rnn_dev_alloc(ctx: *mut rnn_ctx, bytes: usize, out: *mut *mut c_void) -> c_int;
    pub fn rnn_dev_free(ctx: *mut rnn_ctx, p: *mut c_void) -> c_int;
    pub fn rnn_copy_to_device(ctx: *mut rnn_ctx, dst_dev: *mut c_void, src_host: *const c_void, bytes: usize) -> c_int;
    pub fn rnn_copy_to_host(ctx: *mut rnn_ctx, dst_host: *mut c_void, src_dev: *const c_void, bytes: usize) -> c_int;
    pub fn rnn_matmul(ctx: *mut rnn_ctx, m: usize, n: usize, k: usize, a: *const f32, at: c_int, b: *const f32, bt: c_int, c: *mut f32, acc: c_int) -> c_int;
    pub fn rnn_gemm_small_batched(ctx: *mut rnn_ctx, count: usize, m: usize, n: usize, k: usize, a: *const f32, stride_a: usize, at: c_int, b: *const f32, stride_b: usize, bt: c_int, c: *mut f32, stride_c: usize, acc: c_int) -> c_int;
    pub fn rnn_matmul_dw(ctx: *mut rnn_ctx, m: usize, n: usize, k: usize, a: *const f32, b: *const f32, c: *mut f32) -> c_int;
    pub fn rnn_conv_spec_init(sp: *mut rnn_conv_spec, cin: u32, cout: u32, k: u32, stride: u32, pad: u32, h: u32, w: u32) -> c_int;
    pub fn rnn_conv2d_forward(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, x: *const f32, w: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_conv2d_backward_w(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, dy: *const f32, x: *const f32, dw: *mut f32) -> c_int;
    pub fn rnn_conv2d_backward_w_slab_floats(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize) -> usize;
    pub fn rnn_conv2d_backward_w_slabs(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, dy: *const f32, x: *const f32, slabs: *mut f32, nz: *mut c_int) -> c_int;
    pub fn rnn_conv2d_backward_w_noalloc(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, dy: *const f32, x: *const f32, dw: *mut f32) -> c_int;
    pub fn rnn_conv2d_backward_x(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, dy: *const f32, w: *const f32, dx: *mut f32) -> c_int;
    pub fn rnn_conv_packed_floats(sp: *const rnn_conv_spec, dx: c_int, floats: *mut usize) -> c_int;
    pub fn rnn_conv_pack_weights(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, dx: c_int, w: *const f32, wp: *mut f32) -> c_int;
    pub fn rnn_conv2d_forward_packed(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, x: *const f32, w: *const f32, wp: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_conv2d_backward_x_packed(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, dy: *const f32, w: *const f32, wp: *const f32, dx: *mut f32) -> c_int;
    pub fn rnn_conv_packs_create(ctx: *mut rnn_ctx, count: usize, specs: *const rnn_conv_spec, w: *mut *const f32, out: *mut *mut rnn_conv_packs) -> c_int;
    pub fn rnn_conv_packs_update(ctx: *mut rnn_ctx, p: *mut rnn_conv_packs) -> c_int;
    pub fn rnn_conv_packs_get(p: *const rnn_conv_packs, i: usize, dx: c_int) -> *const f32;
    pub fn rnn_conv_packs_destroy(p: *mut rnn_conv_packs);
    pub fn rnn_rel_index(th: u32, tw: u32, mh: u32, mw: u32, idx: *mut u32, nrel: *mut u32) -> c_int;
    pub fn rnn_attn_forward(ctx: *mut rnn_ctx, d: *const rnn_attn_desc, n: usize, q: *const f32, kv: *const f32, tau: *const f32, rel: *const f32, p: *mut f32, o: *mut f32) -> c_int;
    pub fn rnn_attn_backward(ctx: *mut rnn_ctx, d: *const rnn_attn_desc, n: usize, q: *const f32, kv: *const f32, tau: *const f32, p: *const f32, dout: *const f32, dq: *mut f32, dkv: *mut f32, dtau: *mut f32, drel: *mut f32) -> c_int;
    pub fn rnn_attn_backward_ex(ctx: *mut rnn_ctx, d: *const rnn_attn_desc, n: usize, q: *const f32, kv: *const f32, tau: *const f32, p: *const f32, dout: *const f32, dq: *mut f32, dkv: *mut f32, dtau: *mut f32, drel: *mut f32, flags: u32) -> c_int;
    pub fn rnn_linear_forward(ctx: *mut rnn_ctx, rows: usize, fin: usize, fout: usize, x: *const f32, w: *const f32, b: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_linear_forward_residual(ctx: *mut rnn_ctx, rows: usize, fin: usize, fout: usize, x: *const f32, w: *const f32, b: *const f32, y: *mut f32, l: *const f32, mask: *const f32, rpi: usize, out: *mut f32) -> c_int;
    pub fn rnn_linear_backward(ctx: *mut rnn_ctx, rows: usize, fin: usize, fout: usize, dy: *const f32, x: *const f32, w: *const f32, dw: *mut f32, db: *mut f32, dx: *mut f32) -> c_int;
    pub fn rnn_linear_backward_ex(ctx: *mut rnn_ctx, rows: usize, fin: usize, fout: usize, dy: *const f32, x: *const f32, w: *const f32, dw: *mut f32, db: *mut f32, dx: *mut f32, flags: u32) -> c_int;
    pub fn rnn_matmul_host(ctx: *mut rnn_ctx, m: usize, n: usize, k: usize, a: *const f32, at: c_int, b: *const f32, bt: c_int, c: *mut f32, acc: c_int) -> c_int;
    pub fn rnn_gemm_small_batched_host(ctx: *mut rnn_ctx, count: usize, m: usize, n: usize, k: usize, a: *const f32, stride_a: usize, at: c_int, b: *const f32, stride_b: usize, bt: c_int, c: *mut f32, stride_c: usize, acc: c_int) -> c_int;
    pub fn rnn_matmul_dw_host(ctx: *mut rnn_ctx, m: usize, n: usize, k: usize, a: *const f32, b: *const f32, c: *mut f32) -> c_int;
    pub fn rnn_conv2d_forward_host(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, x: *const f32, w: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_conv2d_backward_w_host(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, dy: *const f32, x: *const f32, dw: *mut f32) -> c_int;
    pub fn rnn_conv2d_backward_x_host(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, n: usize, dy: *const f32, w: *const f32, dx: *mut f32) -> c_int;
    pub fn rnn_attn_forward_host(ctx: *mut rnn_ctx, d: *const rnn_attn_desc, n: usize, q: *const f32, kv: *const f32, tau: *const f32, rel: *const f32, p: *mut f32, o: *mut f32) -> c_int;
    pub fn rnn_attn_backward_host(ctx: *mut rnn_ctx, d: *const rnn_attn_desc, n: usize, q: *const f32, kv: *const f32, tau: *const f32, p: *const f32, dout: *const f32, dq: *mut f32, dkv: *mut f32, dtau: *mut f32, drel: *mut f32) -> c_int;
    pub fn rnn_linear_forward_host(ctx: *mut rnn_ctx, rows: usize, fin: usize, fout: usize, x: *const f32, w: *const f32, b: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_linear_backward_host(ctx: *mut rnn_ctx, rows: usize, fin: usize, fout: usize, dy: *const f32, x: *const f32, w: *const f32, dw: *mut f32, db: *mut f32, dx: *mut f32) -> c_int;
    pub fn rnn_bn_forward_train(ctx: *mut rnn_ctx, n: usize, c: usize, hw: usize, x: *const f32, y: *mut f32, gamma: *const f32, beta: *const f32, running_mean: *mut f32, running_var: *mut f32, mean: *mut f32, invstd: *mut f32, momentum: f32, eps: f32, relu: c_int) -> c_int;
    pub fn rnn_bn_forward_eval(ctx: *mut rnn_ctx, n: usize, c: usize, hw: usize, x: *const f32, y: *mut f32, gamma: *const f32, beta: *const f32, running_mean: *const f32, running_var: *const f32, eps: f32, relu: c_int) -> c_int;
    pub fn rnn_bn_backward(ctx: *mut rnn_ctx, n: usize, c: usize, hw: usize, dy: *const f32, relu_out: *const f32, x: *const f32, mean: *const f32, invstd: *const f32, gamma: *const f32, dx: *mut f32, dgamma: *mut f32, dbeta: *mut f32) -> c_int;
    pub fn rnn_relu_back(ctx: *mut rnn_ctx, len: usize, d: *mut f32, y: *const f32) -> c_int;
    pub fn rnn_add(ctx: *mut rnn_ctx, len: usize, a: *mut f32, b: *const f32) -> c_int;
    pub fn rnn_add_relu_back(ctx: *mut rnn_ctx, len: usize, a: *mut f32, b: *const f32, y: *const f32) -> c_int;
    pub fn rnn_add_relu(ctx: *mut rnn_ctx, len: usize, a: *mut f32, b: *const f32) -> c_int;
    pub fn rnn_gap_forward(ctx: *mut rnn_ctx, n: usize, c: usize, hw: usize, x: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_gap_backward(ctx: *mut rnn_ctx, n: usize, c: usize, hw: usize, dy: *const f32, dx: *mut f32) -> c_int;
    pub fn rnn_fc_forward(ctx: *mut rnn_ctx, rows: usize, fin: usize, fout: usize, x: *const f32, w: *const f32, b: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_fc_backward(ctx: *mut rnn_ctx, rows: usize, fin: usize, fout: usize, dy: *const f32, x: *const f32, w: *const f32, dw: *mut f32, db: *mut f32, dx: *mut f32) -> c_int;
    pub fn rnn_softmax_ce(ctx: *mut rnn_ctx, rows: usize, nclass: usize, logits: *const f32, labels: *const u32, smooth: f32, dlogits: *mut f32, loss: *mut f32, correct: *mut u32) -> c_int;
    pub fn rnn_sgd_step(ctx: *mut rnn_ctx, len: usize, v: *mut f32, g: *mut f32, m: *mut f32, lr: f32, momentum: f32, wd: f32) -> c_int;
    pub fn rnn_ln_forward(ctx: *mut rnn_ctx, rows: usize, c: usize, x: *const f32, g: *const f32, b: *const f32, eps: f32, y: *mut f32, xhat: *mut f32, invstd: *mut f32) -> c_int;
    pub fn rnn_ln_backward(ctx: *mut rnn_ctx, rows: usize, c: usize, dy: *const f32, xhat: *const f32, invstd: *const f32, g: *const f32, dx: *mut f32, dg: *mut f32, db: *mut f32) -> c_int;
    pub fn rnn_ln_backward_add(ctx: *mut rnn_ctx, rows: usize, c: usize, dy: *const f32, xhat: *const f32, invstd: *const f32, g: *const f32, add: *const f32, dx: *mut f32, dg: *mut f32, db: *mut f32) -> c_int;
    pub fn rnn_ln_backward_add_ls(ctx: *mut rnn_ctx, rows: usize, c: usize, dy: *const f32, xhat: *const f32, invstd: *const f32, g: *const f32, add: *const f32, dx: *mut f32, dg: *mut f32, db: *mut f32, lsx: *const f32, l: *const f32, mask: *const f32, rpi: usize, lsdx: *mut f32, dl: *mut f32) -> c_int;
    pub fn rnn_layerscale_forward(ctx: *mut rnn_ctx, rows: usize, c: usize, x: *const f32, l: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_layerscale_backward(ctx: *mut rnn_ctx, rows: usize, c: usize, dy: *const f32, x: *const f32, l: *const f32, dx: *mut f32, dl: *mut f32) -> c_int;
    pub fn rnn_drop_layerscale_backward(ctx: *mut rnn_ctx, rows: usize, c: usize, dy: *const f32, x: *const f32, l: *const f32, mask: *const f32, rpi: usize, dx: *mut f32, dl: *mut f32) -> c_int;
    pub fn rnn_block_branch_backward(ctx: *mut rnn_ctx, rows: usize, c: usize, dy: *const f32, a: *const f32, l1: *const f32, m1: *const f32, dwo: *const f32, gamma: *const f32, cm: *const f32, lm: *const f32, m2: *const f32, rpi: usize, da: *mut f32, dl1: *mut f32, ddw: *mut f32, dgamma: *mut f32, dc: *mut f32, dlm: *mut f32) -> c_int;
    pub fn rnn_residual_add_scaled(ctx: *mut rnn_ctx, rows: usize, c: usize, x: *const f32, a: *const f32, l: *const f32, mask: *const f32, rpi: usize, y: *mut f32) -> c_int;
    pub fn rnn_swiglu_forward(ctx: *mut rnn_ctx, rows: usize, h: usize, ab: *const f32, u: *mut f32) -> c_int;
    pub fn rnn_swiglu_backward(ctx: *mut rnn_ctx, rows: usize, h: usize, du: *const f32, ab: *const f32, dab: *mut f32) -> c_int;
    pub fn rnn_dwconv3_forward(ctx: *mut rnn_ctx, n: usize, th: usize, tw: usize, c: usize, x: *const f32, w: *const f32, b: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_dwconv3_backward(ctx: *mut rnn_ctx, n: usize, th: usize, tw: usize, c: usize, dy: *const f32, x: *const f32, w: *const f32, dx: *mut f32, dw: *mut f32, db: *mut f32) -> c_int;
    pub fn rnn_dwconv3_backward_ex(ctx: *mut rnn_ctx, n: usize, th: usize, tw: usize, c: usize, dy: *const f32, x: *const f32, w: *const f32, dx: *mut f32, dw: *mut f32, db: *mut f32, flags: u32) -> c_int;
    pub fn rnn_dwconv3_branch_forward(ctx: *mut rnn_ctx, n: usize, th: usize, tw: usize, c: usize, h: *const f32, w: *const f32, b: *const f32, d: *mut f32, a: *mut f32, gamma: *const f32, x: *const f32, l: *const f32, mask: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_seqpool_forward(ctx: *mut rnn_ctx, n: usize, t: usize, c: usize, x: *const f32, p: *const f32, z: *mut f32, w: *mut f32) -> c_int;
    pub fn rnn_seqpool_backward(ctx: *mut rnn_ctx, n: usize, t: usize, c: usize, dz: *const f32, w: *const f32, x: *const f32, p: *const f32, dx: *mut f32, dp: *mut f32) -> c_int;
    pub fn rnn_soft_targets(ctx: *mut rnn_ctx, n: usize, nf: usize, nc: usize, labels: *const u32, coarse: *const u32, perm: *const u32, lam: *const f32, parent: *const u32, taxo: c_int, eps: f32, sib: f32, tf: *mut f32, tc: *mut f32) -> c_int;
    pub fn rnn_mix_dominant(ctx: *mut rnn_ctx, n: usize, labels: *const u32, perm: *const u32, lam: *const f32, dom: *mut u32) -> c_int;
    pub fn rnn_ce_soft(ctx: *mut rnn_ctx, n: usize, nclass: usize, logits: *const f32, target: *const f32, hard: *const u32, scale: f32, dz: *mut f32, loss: *mut f32, correct: *mut u32) -> c_int;
    pub fn rnn_kl_distill(ctx: *mut rnn_ctx, n: usize, nclass: usize, student: *const f32, teacher: *const f32, temp: f32, scale: f32, dz: *mut f32, loss: *mut f32) -> c_int;
    pub fn rnn_hint_mse(ctx: *mut rnn_ctx, n: usize, c: usize, pred: *const f32, target: *const f32, scale: f32, dz: *mut f32, loss: *mut f32) -> c_int;
    pub fn rnn_build_loss(ctx: *mut rnn_ctx, n: usize, nf: usize, nc: usize, d4: usize, tf: *const f32, tc: *const f32, hard: *const u32, hardc: *const u32, cfg: *const rnn_loss_cfg, io: *const rnn_loss_io, total: *mut f32, ce: *mut f32, correct: *mut u32) -> c_int;
    pub fn rnn_drop_path_forward(ctx: *mut rnn_ctx, n: usize, per: usize, x: *mut f32, p: f32, seed: u64, mask: *mut f32) -> c_int;
    pub fn rnn_drop_path_backward(ctx: *mut rnn_ctx, n: usize, per: usize, dy: *mut f32, mask: *const f32) -> c_int;
    pub fn rnn_drop_path_masks(ctx: *mut rnn_ctx, count: usize, n: usize, p: *const f32, seeds: *const u64, masks: *mut *mut float  const) -> c_int;
    pub fn rnn_axpy_cols(ctx: *mut rnn_ctx, rows: usize, c: usize, y: *mut f32, l: *const f32, x: *const f32) -> c_int;
    pub fn rnn_token_merge(ctx: *mut rnn_ctx, n: usize, th: usize, c: usize, z: *const f32, y: *mut f32) -> c_int;
    pub fn rnn_token_merge_backward(ctx: *mut rnn_ctx, n: usize, th: usize, c: usize, dy: *const f32, dz: *mut f32) -> c_int;
    pub fn rnn_taxo_head_combine(ctx: *mut rnn_ctx, n: usize, nf: usize, nc: usize, parent: *const u32, zf: *mut f32, zc: *const f32) -> c_int;
    pub fn rnn_taxo_head_combine_backward(ctx: *mut rnn_ctx, n: usize, nf: usize, nc: usize, parent: *const u32, dzf: *const f32, dzc: *const f32, dc: *mut f32) -> c_int;
    pub fn rnn_nchw_to_tokens(ctx: *mut rnn_ctx, n: usize, c: usize, hw: usize, x: *const f32, t: *mut f32) -> c_int;
    pub fn rnn_tokens_to_nchw(ctx: *mut rnn_ctx, n: usize, c: usize, hw: usize, t: *const f32, x: *mut f32) -> c_int;
    pub fn rnn_cifar_batch_train(ctx: *mut rnn_ctx, images: *const uint8_t, fine: *const uint8_t, coarse: *const uint8_t, nimg: usize, idx: *const u32, bs: usize, pad: usize, ra_mag: f32, ra_n: usize, erase: f32, erase_side: usize, seed: u64, out: *mut f32, labels: *mut u32, coarse_out: *mut u32) -> c_int;
    pub fn rnn_cifar_batch_eval(ctx: *mut rnn_ctx, images: *const uint8_t, fine: *const uint8_t, nimg: usize, start: usize, bs: usize, flip: c_int, out: *mut f32, labels: *mut u32) -> c_int;
    pub fn rnn_fnv1a_bytes(hash: u64, bytes: *const uint8_t, n: usize) -> u64;
    pub fn rnn_fnv1a_f32(hash: u64, values: *const f32, n: usize) -> u64;
    pub fn rnn_rng_seed(seed: u64, state: *mut u64) -> c_int;
    pub fn rnn_rng_next_u64(state: *mut u64) -> u64;
    pub fn rnn_rng_normal_vec(state: *mut u64, n: usize, scale: f32, out: *mut f32) -> c_int;
    pub fn rnn_rng_trunc_normal(state: *mut u64, n: usize, std_: f32, out: *mut f32) -> c_int;
    pub fn rnn_mix_plan(rng_state: *mut u64, bs: usize, alpha_mix: f32, alpha_cut: f32, sw: f32, perm: *mut u32, lam: *mut f32, cut: *mut c_int, l: *mut f32, rect: *mut c_int) -> c_int;
    pub fn rnn_mix_apply(ctx: *mut rnn_ctx, x: *const f32, out: *mut f32, bs: usize, perm: *const u32, cut: c_int, l: f32, rect: *const c_int) -> c_int;
    pub fn rnn_newton_schulz(ctx: *mut rnn_ctx, count: usize, rows: usize, cols: usize, steps: usize, g: *mut f32, stride: usize) -> c_int;
    pub fn rnn_optim_create(ctx: *mut rnn_ctx, muon: c_int, ns_steps: usize, out: *mut *mut rnn_optim) -> c_int;
    pub fn rnn_optim_destroy(opt: *mut rnn_optim) -> c_int;
    pub fn rnn_optim_set(opt: *mut rnn_optim, mom: f32, b1: f32, b2: f32, eps: f32, t: usize) -> c_int;
    pub fn rnn_optim_t(opt: *const rnn_optim) -> usize;
    pub fn rnn_optim_step(opt: *mut rnn_optim, nparam: usize, params: *const rnn_param, lr: f32, wd: f32) -> c_int;
    pub fn rnn_clip_grad_norm(ctx: *mut rnn_ctx, len: usize, g: *mut f32, max: f32, norm: *mut f32) -> c_int;
    pub fn rnn_clip_params(ctx: *mut rnn_ctx, nparam: usize, params: *const rnn_param, max: f32, norm: *mut f32) -> c_int;
    pub fn rnn_ema_update(ctx: *mut rnn_ctx, len: usize, w: *mut f32, v: *const f32, d: f32) -> c_int;
    pub fn rnn_ema_update_params(ctx: *mut rnn_ctx, nparam: usize, w: *mut *mut float  const, params: *const rnn_param, d: f32) -> c_int;
    pub fn rnn_powi_f32(a: f32, b: c_int) -> f32;
    pub fn rnn_lr_at(peak: f32, lo: f32, step: usize, total: usize, warm: usize) -> f32;
    pub fn rnn_resnet_create(ctx: *mut rnn_ctx, depth_n: usize, width: usize, nclass: usize, seed: u64, out: *mut *mut rnn_resnet) -> c_int;
    pub fn rnn_resnet_destroy(net: *mut rnn_resnet) -> c_int;
    pub fn rnn_resnet_num_params(net: *const rnn_resnet) -> usize;
    pub fn rnn_resnet_num_buffers(net: *const rnn_resnet) -> usize;
    pub fn rnn_resnet_num_tensors(net: *const rnn_resnet) -> usize;
    pub fn rnn_resnet_tensor_len(net: *const rnn_resnet, i: usize, len: *mut usize, decay: *mut c_int) -> c_int;
    pub fn rnn_resnet_copy(net: *mut rnn_resnet, which: c_int, dst: *mut f32, src: *const f32) -> c_int;
    pub fn rnn_resnet_forward(net: *mut rnn_resnet, n: usize, h: usize, w: usize, x: *const f32, train: c_int, logits: *mut f32) -> c_int;
    pub fn rnn_resnet_backward(net: *mut rnn_resnet, dlogits: *const f32) -> c_int;
    pub fn rnn_resnet_step(net: *mut rnn_resnet, lr: f32, momentum: f32, wd: f32) -> c_int;
    pub fn rnn_resnet_train_step(net: *mut rnn_resnet, n: usize, h: usize, w: usize, x: *const f32, labels: *const u32, smooth: f32, lr: f32, momentum: f32, wd: f32, loss: *mut f32, correct: *mut u32) -> c_int;
    pub fn rnn_resnet_inputs(net: *mut rnn_resnet, n: usize, h: usize, w: usize, x: *mut *mut f32, labels: *mut *mut u32) -> c_int;
    pub fn rnn_resnet_logits(net: *mut rnn_resnet, logits: *mut f32) -> c_int;
    pub fn rnn_resnet_set_graph(net: *mut rnn_resnet, on: c_int) -> c_int;
    pub fn rnn_resnet_graph_state(net: *const rnn_resnet, why: *mut *const c_char) -> c_int;
    pub fn rnn_resnet_flops(net: *const rnn_resnet, h: usize, w: usize) -> u64;
    pub fn rnn_dbg_resnet_buffer(net: *mut rnn_resnet, block: usize, which: c_int, ptr: *mut *const f32, len: *mut usize) -> c_int;
    pub fn rnn_dbg_resnet_dw_group(net: *mut rnn_resnet, launch: c_int, flops: *mut f64) -> c_int;
    pub fn rnn_dbg_im2col(ctx: *mut rnn_ctx, sp: *const rnn_conv_spec, x_img: *const f32, col: *mut f32) -> c_int;
    pub fn rnn_dbg_pack_a(ctx: *mut rnn_ctx, a: *const f32, m: usize, k: usize, transposed: c_int, out: *mut f32) -> c_int;
    pub fn rnn_dbg_pack_b(ctx: *mut rnn_ctx, b: *const f32, n: usize, k: usize, transposed: c_int, out: *mut f32) -> c_int;
    pub fn rnn_dbg_rel_index(ctx: *mut rnn_ctx, th: u32, tw: u32, mh: u32, mw: u32, idx: *mut u32) -> c_int;
}

// Hand-written safe layer (src/safe.rs): the reference's call-site
// signatures over the *_host entry points.
pub mod safe;

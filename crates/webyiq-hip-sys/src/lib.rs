//! FFI binding of the MI355X (gfx950) int4 x int8 linear-layer library.
//!
//! `extern "C"` mirrors `include/webyiq_q4q8.h` one to one (names, argument
//! order and types; a CPU test of the repository checks the two against each
//! other).  The safe layer below maps the reference engine's operator calls
//! onto it with the engine's error convention, `Result<_, String>`:
//!
//! | webyIQ (crates/engine/src/graph.rs)           | here                       |
//! |-----------------------------------------------|----------------------------|
//! | `Builder::quant`   (graph.rs:216-222)          | [`quant`]                  |
//! | `Builder::gemv`    (graph.rs:190-198)          | [`gemv`]                   |
//! | `Builder::gemm`    (graph.rs:200-205)          | [`gemm`]                   |
//! | `Builder::matmul`  (graph.rs:207-214)          | [`matmul`]                 |
//! | quant -> matmul pairs (graph.rs:266+269, ...)  | [`quant_gemv`]             |
//! | `head_ops` gemv + argmax (graph.rs:476-486)    | [`lm_head_argmax`]         |
//!
//! Every pointer is device memory (hipMalloc) owned by the caller; every
//! call is asynchronous on `stream` (a hipStream_t, null = default stream).

use std::ffi::{c_char, c_void, CStr};

pub const WQ_ABI_VERSION: i32 = 2;

pub const WQ_OK: i32 = 0;
pub const WQ_EINVAL: i32 = -1;
pub const WQ_ESHAPE: i32 = -2;
pub const WQ_EALIGN: i32 = -3;
pub const WQ_EHIP: i32 = -4;
pub const WQ_EWORKSPACE: i32 = -5;

pub const WQ_MODE_STORE: i32 = 0;
pub const WQ_MODE_ACCUMULATE: i32 = 1;
pub const WQ_MODE_SILU_MUL: i32 = 2;

pub const WQ_PATH_DECODE: i32 = 0;
pub const WQ_PATH_SPEC: i32 = 1;
pub const WQ_PATH_PREFILL: i32 = 2;

/// The step parameters the kernels read when they run (`wq_params`; the
/// engine's `Params` uniform, gemm_q4q8.wgsl:8-13), passed as a pointer to
/// device memory: the engine's `params` buffer (graph.rs:413-416), written
/// per step by the host (lib.rs:312-314) or by the GPU (lib.rs:325).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct WqParams {
    pub pos: u32,
    pub seq_len: u32,
    pub m: u32,
    pub slot: u32,
}

extern "C" {
    pub fn wq_last_error() -> *const c_char;
    pub fn wq_abi_version() -> i32;
    pub fn wq_quant_act(stream: *mut c_void, x: *const f32, norm_w: *const f32, eps: f32, m: i64, k: i64,
                        ga: i32, g: i32, xq: *mut i8, dx: *mut f32, xs: *mut i32) -> i32;
    pub fn wq_gemv(stream: *mut c_void, wq: *const u32, ws: *const u32, n: i64, k: i64, g: i32, xq: *const i8,
                   dx: *const f32, xs: *const i32, m: i64, ga: i32, mode: i32, y: *mut f32) -> i32;
    pub fn wq_quant_gemv(stream: *mut c_void, x: *const f32, norm_w: *const f32, eps: f32, wq: *const u32,
                         ws: *const u32, n: i64, k: i64, g: i32, m: i64, mode: i32, xq: *mut i8, dx: *mut f32,
                         xs: *mut i32, y: *mut f32) -> i32;
    pub fn wq_gemm(stream: *mut c_void, wq: *const u32, ws: *const u32, n: i64, k: i64, g: i32, xq: *const i8,
                   dx: *const f32, xs: *const i32, m: i64, ga: i32, mode: i32, y: *mut f32,
                   params: *const WqParams, workspace: *mut c_void, workspace_bytes: usize) -> i32;
    pub fn wq_gemm_workspace_bytes(n: i64, k: i64, g: i32, m: i64, ga: i32, mode: i32) -> usize;
    pub fn wq_matmul(stream: *mut c_void, path: i32, wq: *const u32, ws: *const u32, n: i64, k: i64, g: i32,
                     xq: *const i8, dx: *const f32, xs: *const i32, m: i64, ga: i32, mode: i32,
                     y: *mut f32, params: *const WqParams) -> i32;
    pub fn wq_argmax(stream: *mut c_void, logits: *const f32, m: i64, v: i64, ids: *const u32,
                     tok_out: *mut u32) -> i32;
    pub fn wq_lm_head_argmax(stream: *mut c_void, wq: *const u32, ws: *const u32, v: i64, k: i64, g: i32,
                             xq: *const i8, dx: *const f32, xs: *const i32, m: i64, ga: i32, ids: *const u32,
                             logits: *mut f32, tok_out: *mut u32, workspace: *mut c_void,
                             workspace_bytes: usize) -> i32;
    pub fn wq_lm_head_argmax_noalloc(stream: *mut c_void, wq: *const u32, ws: *const u32, v: i64, k: i64,
                                     g: i32, xq: *const i8, dx: *const f32, xs: *const i32, m: i64, ga: i32,
                                     ids: *const u32, logits: *mut f32, tok_out: *mut u32) -> i32;
    pub fn wq_lm_head_noalloc_reset(stream: *mut c_void) -> i32;
    pub fn wq_lm_head_workspace_bytes() -> usize;
    pub fn wq_workspace_clear(stream: *mut c_void, workspace: *mut c_void, bytes: usize) -> i32;
    pub fn wq_embed(stream: *mut c_void, eq: *const u32, es: *const u32, v: i64, k: i64, g: i32,
                    tok: *const u32, m: i64, x: *mut f32) -> i32;
    pub fn wq_gather_rows(stream: *mut c_void, sq: *const u32, ss: *const u32, v: i64, k: i64, g: i32,
                          ids: *const u32, r: i64, dq: *mut u32, ds: *mut u32) -> i32;
    pub fn wq_mtp_in(stream: *mut c_void, emb: *const f32, x: *const f32, norm_f: *const f32,
                     norm_e: *const f32, norm_h: *const f32, eps: f32, m: i64, k: i64, xq: *mut i8,
                     dx: *mut f32, xs: *mut i32) -> i32;
    pub fn wq_attn_combine(stream: *mut c_void, part: *const f32, m: i64, h: i64, d: i64, nch: i64, pos: i64,
                           gate: *const f32, gate_stride: i64, xq: *mut i8, dx: *mut f32, xs: *mut i32,
                           params: *const WqParams) -> i32;
    pub fn wq_gemv_debug_acc(stream: *mut c_void, wq: *const u32, ws: *const u32, n: i64, k: i64, g: i32,
                             xq: *const i8, dx: *const f32, xs: *const i32, m: i64, ga: i32, mode: i32,
                             y: *mut f32, acc: *mut i32) -> i32;
    pub fn wq_gemm_debug_acc(stream: *mut c_void, wq: *const u32, ws: *const u32, n: i64, k: i64, g: i32,
                             xq: *const i8, dx: *const f32, xs: *const i32, m: i64, ga: i32, mode: i32,
                             y: *mut f32, acc: *mut i32) -> i32;
}

/// The engine's error convention: `Ok(())`, or `Err` with `wq_last_error()`.
pub fn check(rc: i32) -> Result<(), String> {
    if rc == WQ_OK {
        Ok(())
    } else {
        let msg = unsafe { CStr::from_ptr(wq_last_error()) }.to_string_lossy().into_owned();
        Err(format!("[{rc}] {msg}"))
    }
}

/// A HIP stream (hipStream_t); the null stream is the default stream.
#[derive(Clone, Copy, Debug)]
pub struct Stream(pub *mut c_void);

/// A packed int4 linear weight on the device: `{name}.q` u32 [rows, K/8] and
/// `{name}.s` u32 [rows, K/G] (tools/convert.py:8-12), the engine's
/// `weights["{name}.q"] / ["{name}.s"]` buffers (graph.rs:186-193).
#[derive(Clone, Copy, Debug)]
pub struct Q4Weight {
    pub q: *const u32,
    pub s: *const u32,
    pub rows: i64,
    pub k: i64,
    pub g: i32,
}

/// Quantised activations: xq i8 [m, k], dx f32 [m, k/ga], xs i32 [m, k/min(g, ga)].
/// The reference packs (dx, dx * sum) as vec2<f32> per group (quant.wgsl:41-61);
/// this layout keeps the scale and the exact integer group sums apart.
#[derive(Clone, Copy, Debug)]
pub struct Acts {
    pub xq: *mut i8,
    pub dx: *mut f32,
    pub xs: *mut i32,
    pub m: i64,
    pub k: i64,
    pub ga: i32,
}

/// `Builder::quant`: per-token (ga = k) or per-32 int8 quantisation of x f32
/// [m, k], with the RMSNorm prologue when `norm` is non-null.
///
/// # Safety
/// All pointers must be device memory of the documented sizes.
pub unsafe fn quant(st: Stream, x: *const f32, norm: *const f32, eps: f32, g: i32, a: &Acts) -> Result<(), String> {
    check(wq_quant_act(st.0, x, norm, eps, a.m, a.k, a.ga, g, a.xq, a.dx, a.xs))
}

/// `Builder::gemv`: decode GEMV for m <= 8 tokens (mode STORE / ACCUMULATE /
/// SILU_MUL; `n` output rows, 2n weight rows in SILU_MUL).
///
/// # Safety
/// All pointers must be device memory of the documented sizes.
pub unsafe fn gemv(st: Stream, w: &Q4Weight, n: i64, a: &Acts, mode: i32, y: *mut f32) -> Result<(), String> {
    check(wq_gemv(st.0, w.q, w.s, n, w.k, w.g, a.xq, a.dx, a.xs, a.m, a.ga, mode, y))
}

/// `Builder::gemm`: prefill GEMM on int8 MFMA, any token count.  With a
/// non-null `params` (the engine's params buffer), `a.m` is the capacity and
/// the kernel covers `params.m` tokens, read when it runs.  `workspace`
/// (null, or `wq_gemm_workspace_bytes` bytes zeroed once) lets the library
/// split K between workgroup pairs.
///
/// # Safety
/// All pointers must be device memory of the documented sizes.
pub unsafe fn gemm(st: Stream, w: &Q4Weight, n: i64, a: &Acts, mode: i32, y: *mut f32,
                   params: *const WqParams, workspace: *mut c_void,
                   workspace_bytes: usize) -> Result<(), String> {
    check(wq_gemm(st.0, w.q, w.s, n, w.k, w.g, a.xq, a.dx, a.xs, a.m, a.ga, mode, y, params, workspace,
                  workspace_bytes))
}

/// `Builder::matmul`: the engine's `Path` picks the GEMV or the GEMM.
///
/// # Safety
/// All pointers must be device memory of the documented sizes.
pub unsafe fn matmul(st: Stream, path: i32, w: &Q4Weight, n: i64, a: &Acts, mode: i32,
                     y: *mut f32, params: *const WqParams) -> Result<(), String> {
    check(wq_matmul(st.0, path, w.q, w.s, n, w.k, w.g, a.xq, a.dx, a.xs, a.m, a.ga, mode, y, params))
}

/// A quant -> decode matmul pair of the layer in one call (one launch for
/// m <= 2); the quantised activations are written to `a` (per token).
///
/// # Safety
/// All pointers must be device memory of the documented sizes.
pub unsafe fn quant_gemv(st: Stream, x: *const f32, norm: *const f32, eps: f32, w: &Q4Weight, n: i64,
                         a: &Acts, mode: i32, y: *mut f32) -> Result<(), String> {
    check(wq_quant_gemv(st.0, x, norm, eps, w.q, w.s, n, w.k, w.g, a.m, mode, a.xq, a.dx, a.xs, y))
}

/// `head_ops`' gemv + argmax in one launch: the greedy token per row, ids
/// mapped through `ids` when non-null (the draft vocabulary).
///
/// # Safety
/// All pointers must be device memory of the documented sizes; `workspace`
/// holds `wq_lm_head_workspace_bytes()` bytes, zeroed once.
pub unsafe fn lm_head_argmax(st: Stream, w: &Q4Weight, a: &Acts, ids: *const u32, logits: *mut f32,
                             tok_out: *mut u32, workspace: *mut c_void) -> Result<(), String> {
    check(wq_lm_head_argmax(st.0, w.q, w.s, w.rows, w.k, w.g, a.xq, a.dx, a.xs, a.m, a.ga, ids, logits,
                            tok_out, workspace, wq_lm_head_workspace_bytes()))
}

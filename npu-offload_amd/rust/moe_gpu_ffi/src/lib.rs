//! Rust binding of libmoe_gpu, the MI355X routed-MoE expert tier (include/moe_gpu.h), for the reference engine
//! (track2_opt/solar_engine).  `ffi` mirrors the C declarations; `GpuTier` and `GpuModel` wrap a context the way the
//! engine wraps a chip (chip.rs:96-143): one owner thread, errors as `Result` (the engine's chip replies are
//! eyre::Result, chip.rs:59; `Error` converts into eyre::Report with `?`).
use std::ffi::CStr;
use std::fmt;
use std::os::raw::{c_char, c_int, c_uint, c_void};

pub mod ffi {
    use super::*;

    #[repr(C)]
    pub struct MoeGpu {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct MoeHead {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct MoeModel {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct MoeSt {
        _private: [u8; 0],
    }
    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct MoeModelConfig {
        pub h: c_int,
        pub n_q_heads: c_int,
        pub n_kv_heads: c_int,
        pub head_dim: c_int,
        pub f: c_int,
        pub e: c_int,
        pub topk: c_int,
        pub n_shared: c_int,
        pub n_layers: c_int,
        pub vocab: c_int,
        pub max_ctx: c_int,
        pub eps: f32,
        pub route_rule: c_int,
        pub argmax_rule: c_int,
    }

    pub const MOE_GPU_ACCUMULATE: c_uint = 1;
    pub const MOE_GPU_INT8: c_uint = 2;
    pub const MOE_GPU_OPT_ROUTE_RULE: c_int = 10;
    pub const MOE_GPU_ROUTE_SOFTMAX: c_int = 0;
    pub const MOE_GPU_ROUTE_SIGMOID: c_int = 1;
    pub const MOE_HEAD_ARGMAX_FP32: c_int = 0;
    pub const MOE_HEAD_ARGMAX_BF16: c_int = 1;

    extern "C" {
        pub fn moe_gpu_create(device: c_int, h: c_int, f: c_int, e: c_int, topk: c_int, n_shared: c_int,
                              n_layers: c_int, max_tokens: c_int, out: *mut *mut MoeGpu) -> c_int;
        pub fn moe_gpu_destroy(ctx: *mut MoeGpu);
        pub fn moe_gpu_last_error(ctx: *const MoeGpu) -> *const c_char;
        pub fn moe_gpu_set_stream(ctx: *mut MoeGpu, stream: *mut c_void) -> c_int;
        pub fn moe_gpu_synchronize(ctx: *mut MoeGpu) -> c_int;
        pub fn moe_gpu_set_option(ctx: *mut MoeGpu, opt: c_int, value: c_int) -> c_int;
        pub fn moe_gpu_load_expert(ctx: *mut MoeGpu, layer: c_int, e: c_int, g: *const u16, u: *const u16,
                                   d: *const u16) -> c_int;
        pub fn moe_gpu_load_shared(ctx: *mut MoeGpu, layer: c_int, s: c_int, g: *const u16, u: *const u16,
                                   d: *const u16) -> c_int;
        pub fn moe_gpu_load_router(ctx: *mut MoeGpu, layer: c_int, wr: *const u16, bias: *const f32) -> c_int;
        pub fn moe_gpu_load_expert_q8(ctx: *mut MoeGpu, layer: c_int, e: c_int, q: *const i8, sc: *const f32) -> c_int;
        pub fn moe_gpu_quantize_experts(ctx: *mut MoeGpu, layer: c_int, e0: c_int, e1: c_int) -> c_int;
        pub fn moe_gpu_route(ctx: *mut MoeGpu, layer: c_int, t: c_int, x: *const u16, keep: c_int, ids: *mut i32,
                             gates: *mut f32, logits: *mut f32) -> c_int;
        pub fn moe_gpu_moe(ctx: *mut MoeGpu, layer: c_int, t: c_int, x: *const u16, ids: *const i32,
                           gates: *const f32, keep: c_int, with_shared: c_int, flags: c_uint, out: *mut f32) -> c_int;
        pub fn moe_gpu_layer(ctx: *mut MoeGpu, layer: c_int, t: c_int, x: *const u16, keep: c_int, flags: c_uint,
                             out: *mut f32, ids: *mut i32, gates: *mut f32) -> c_int;

        pub fn moe_head_load(h: *mut MoeHead, w_lm: *const u16, w_final: *const u16) -> c_int;
        pub fn moe_head_last_error(h: *const MoeHead) -> *const c_char;

        pub fn moe_model_create(device: c_int, cfg: *const MoeModelConfig, out: *mut *mut MoeModel) -> c_int;
        pub fn moe_model_destroy(m: *mut MoeModel);
        pub fn moe_model_last_error(m: *const MoeModel) -> *const c_char;
        pub fn moe_model_experts(m: *mut MoeModel) -> *mut MoeGpu;
        pub fn moe_model_head(m: *mut MoeModel) -> *mut MoeHead;
        pub fn moe_model_load_layer(m: *mut MoeModel, layer: c_int, in_norm: *const u16, wq: *const u16,
                                    wk: *const u16, wv: *const u16, wo: *const u16, post_norm: *const u16) -> c_int;
        pub fn moe_model_load_embedding(m: *mut MoeModel, emb: *const u16) -> c_int;
        pub fn moe_model_load_rope(m: *mut MoeModel, cos_tab: *const u16, sin_tab: *const u16) -> c_int;
        pub fn moe_model_step(m: *mut MoeModel, token: c_int, pos: c_int, next: *mut i32, best: *mut f32) -> c_int;
        pub fn moe_st_open(dir: *const c_char, out: *mut *mut MoeSt) -> c_int;
        pub fn moe_st_close(st: *mut MoeSt);
        pub fn moe_st_last_error(st: *const MoeSt) -> *const c_char;
        pub fn moe_st_load_moe_layer(st: *const MoeSt, ctx: *mut MoeGpu, model_layer: c_int, tier_layer: c_int,
                                     experts: *const i32, n: c_int) -> c_int;
        pub fn moe_st_load_model(st: *const MoeSt, m: *mut MoeModel) -> c_int;
        pub fn moe_placement_read(path: *const c_char, layer: c_int, tier: c_int, ids: *mut i32, cap: c_int,
                                  n: *mut c_int) -> c_int;
    }
}

/// A libmoe_gpu call that returned a negative status, with the library's message.
#[derive(Debug, Clone)]
pub struct Error {
    pub code: i32,
    pub msg: String,
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "moe_gpu error {}: {}", self.code, self.msg)
    }
}
impl std::error::Error for Error {}

fn cstr(p: *const c_char) -> String {
    if p.is_null() {
        return String::new();
    }
    unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
}

fn check(rc: c_int, msg: impl FnOnce() -> String) -> Result<(), Error> {
    if rc == 0 { Ok(()) } else { Err(Error { code: rc, msg: msg() }) }
}

/// One GPU expert tier holding every expert of every layer in HBM: the engine's chip (chip.rs:96-143) with the NPU
/// tables replaced by HIP tables.  Used from one host thread.
pub struct GpuTier {
    ctx: *mut ffi::MoeGpu,
    owned: bool,
    pub h: usize,
    pub k: usize,
}

impl GpuTier {
    pub fn new(device: i32, h: usize, f: usize, e: usize, k: usize, n_shared: usize, layers: usize,
               max_tokens: usize) -> Result<Self, Error> {
        let mut ctx = std::ptr::null_mut();
        let rc = unsafe {
            ffi::moe_gpu_create(device, h as c_int, f as c_int, e as c_int, k as c_int, n_shared as c_int,
                                layers as c_int, max_tokens as c_int, &mut ctx)
        };
        check(rc, || cstr(unsafe { ffi::moe_gpu_last_error(std::ptr::null()) }))?;
        Ok(Self { ctx, owned: true, h, k })
    }
    fn ok(&self, rc: c_int) -> Result<(), Error> {
        check(rc, || cstr(unsafe { ffi::moe_gpu_last_error(self.ctx) }))
    }
    /// Solar's own routing rule (host.rs:119-128): sigmoid scores, the bias selects only.
    pub fn use_sigmoid_routing(&mut self) -> Result<(), Error> {
        self.ok(unsafe { ffi::moe_gpu_set_option(self.ctx, ffi::MOE_GPU_OPT_ROUTE_RULE, ffi::MOE_GPU_ROUTE_SIGMOID) })
    }
    /// place_expert (host.rs:144-153) / the chip table upload (chip.rs:208-233): g, u [F,H], d [H,F] bf16.
    pub fn load_expert(&mut self, layer: usize, e: usize, g: &[u16], u: &[u16], d: &[u16]) -> Result<(), Error> {
        self.ok(unsafe { ffi::moe_gpu_load_expert(self.ctx, layer as c_int, e as c_int, g.as_ptr(), u.as_ptr(), d.as_ptr()) })
    }
    pub fn load_shared(&mut self, layer: usize, s: usize, g: &[u16], u: &[u16], d: &[u16]) -> Result<(), Error> {
        self.ok(unsafe { ffi::moe_gpu_load_shared(self.ctx, layer as c_int, s as c_int, g.as_ptr(), u.as_ptr(), d.as_ptr()) })
    }
    pub fn load_router(&mut self, layer: usize, wr: &[u16], bias: Option<&[f32]>) -> Result<(), Error> {
        let b = bias.map_or(std::ptr::null(), |b| b.as_ptr());
        self.ok(unsafe { ffi::moe_gpu_load_router(self.ctx, layer as c_int, wr.as_ptr(), b) })
    }
    /// place_expert_q8 (host.rs:163-179) on the device: quantise resident bf16 experts [e0, e1) with quant_row's rule.
    pub fn quantize(&mut self, layer: usize, e0: usize, e1: usize) -> Result<(), Error> {
        self.ok(unsafe { ffi::moe_gpu_quantize_experts(self.ctx, layer as c_int, e0 as c_int, e1 as c_int) })
    }
    /// Router GEMV + top-k (ids / gates [T, k]).
    pub fn route(&mut self, layer: usize, x: &[u16], keep: usize, ids: &mut [i32], gates: &mut [f32]) -> Result<(), Error> {
        let t = x.len() / self.h;
        self.ok(unsafe {
            ffi::moe_gpu_route(self.ctx, layer as c_int, t as c_int, x.as_ptr(), keep as c_int, ids.as_mut_ptr(),
                               gates.as_mut_ptr(), std::ptr::null_mut())
        })
    }
    /// ck_moe3 / moe_cpu semantics: out += sum_r gates[r] * expert_{ids[r]}(x) (+ the shared experts), T tokens.
    pub fn moe(&mut self, layer: usize, x: &[u16], ids: &[i32], gates: &[f32], keep: usize, with_shared: bool,
               int8: bool, out: &mut [f32]) -> Result<(), Error> {
        let t = x.len() / self.h;
        let flags = ffi::MOE_GPU_ACCUMULATE | if int8 { ffi::MOE_GPU_INT8 } else { 0 };
        self.ok(unsafe {
            ffi::moe_gpu_moe(self.ctx, layer as c_int, t as c_int, x.as_ptr(), ids.as_ptr(), gates.as_ptr(),
                             keep as c_int, with_shared as c_int, flags, out.as_mut_ptr())
        })
    }
    /// Route + experts + shared + combine with ids never leaving the device; ids / gates come back for statistics.
    pub fn layer(&mut self, layer: usize, x: &[u16], keep: usize, out: &mut [f32], ids: &mut [i32],
                 gates: &mut [f32]) -> Result<(), Error> {
        let t = x.len() / self.h;
        self.ok(unsafe {
            ffi::moe_gpu_layer(self.ctx, layer as c_int, t as c_int, x.as_ptr(), keep as c_int, 0, out.as_mut_ptr(),
                               ids.as_mut_ptr(), gates.as_mut_ptr())
        })
    }
}

impl Drop for GpuTier {
    fn drop(&mut self) {
        if self.owned {
            unsafe { ffi::moe_gpu_destroy(self.ctx) }
        }
    }
}

/// The whole decode step on the GPU (main.rs:372-387): every layer's weights resident, one call per token.
pub struct GpuModel {
    m: *mut ffi::MoeModel,
}

impl GpuModel {
    pub fn new(device: i32, cfg: ffi::MoeModelConfig) -> Result<Self, Error> {
        let mut m = std::ptr::null_mut();
        let rc = unsafe { ffi::moe_model_create(device, &cfg, &mut m) };
        check(rc, || cstr(unsafe { ffi::moe_model_last_error(std::ptr::null()) }))?;
        Ok(Self { m })
    }
    fn ok(&self, rc: c_int) -> Result<(), Error> {
        check(rc, || cstr(unsafe { ffi::moe_model_last_error(self.m) }))
    }
    /// The MoE tier inside the model (load routers and experts through it); owned by the model.
    pub fn experts(&mut self) -> GpuTier {
        GpuTier { ctx: unsafe { ffi::moe_model_experts(self.m) }, owned: false, h: 0, k: 0 }
    }
    /// model.layers.{l}: input_layernorm, q/k/v/o_proj, post_attention_layernorm (Weights::layer, host.rs:113).
    pub fn load_layer(&mut self, l: usize, in_norm: &[u16], wq: &[u16], wk: &[u16], wv: &[u16], wo: &[u16],
                      post_norm: &[u16]) -> Result<(), Error> {
        self.ok(unsafe {
            ffi::moe_model_load_layer(self.m, l as c_int, in_norm.as_ptr(), wq.as_ptr(), wk.as_ptr(), wv.as_ptr(),
                                      wo.as_ptr(), post_norm.as_ptr())
        })
    }
    pub fn load_embedding(&mut self, emb: &[u16]) -> Result<(), Error> {
        self.ok(unsafe { ffi::moe_model_load_embedding(self.m, emb.as_ptr()) })
    }
    /// rope_cos.bin / rope_sin.bin (main.rs:4): [max_ctx, head_dim] bf16.
    pub fn load_rope(&mut self, cos: &[u16], sin: &[u16]) -> Result<(), Error> {
        self.ok(unsafe { ffi::moe_model_load_rope(self.m, cos.as_ptr(), sin.as_ptr()) })
    }
    /// model.norm.weight and lm_head.weight.
    pub fn load_head(&mut self, w_lm: &[u16], w_final: &[u16]) -> Result<(), Error> {
        let h = unsafe { ffi::moe_model_head(self.m) };
        let rc = unsafe { ffi::moe_head_load(h, w_lm.as_ptr(), w_final.as_ptr()) };
        check(rc, || cstr(unsafe { ffi::moe_head_last_error(h) }))
    }
    /// Model::step (main.rs:372-387): the next greedy token after `token` at position `pos`.
    pub fn step(&mut self, token: usize, pos: usize) -> Result<usize, Error> {
        let mut next = 0i32;
        let mut best = 0f32;
        self.ok(unsafe { ffi::moe_model_step(self.m, token as c_int, pos as c_int, &mut next, &mut best) })?;
        Ok(next as usize)
    }
}

impl Drop for GpuModel {
    fn drop(&mut self) {
        unsafe { ffi::moe_model_destroy(self.m) }
    }
}

/// The model directory's safetensors files, memory-mapped (Weights::open, host.rs:82-99), for loading a tier layer or
/// a whole GpuModel by the engine's tensor names.
pub struct Weights {
    st: *mut ffi::MoeSt,
}

impl Weights {
    pub fn open(dir: &str) -> Result<Self, Error> {
        let c = std::ffi::CString::new(dir).map_err(|_| Error { code: -1, msg: "NUL in path".into() })?;
        let mut st = std::ptr::null_mut();
        let rc = unsafe { ffi::moe_st_open(c.as_ptr(), &mut st) };
        check(rc, || cstr(unsafe { ffi::moe_st_last_error(std::ptr::null()) }))?;
        Ok(Self { st })
    }
    fn ok(&self, rc: c_int) -> Result<(), Error> {
        check(rc, || cstr(unsafe { ffi::moe_st_last_error(self.st) }))
    }
    /// Router, bias, shared experts and the listed routed experts (None: all) of model layer `l` into tier layer `tl`.
    pub fn load_moe_layer(&self, tier: &mut GpuTier, l: usize, tl: usize, experts: Option<&[i32]>) -> Result<(), Error> {
        let (p, n) = experts.map_or((std::ptr::null(), -1), |e| (e.as_ptr(), e.len() as c_int));
        self.ok(unsafe { ffi::moe_st_load_moe_layer(self.st, tier.ctx, l as c_int, tl as c_int, p, n) })
    }
    pub fn load_model(&self, m: &mut GpuModel) -> Result<(), Error> {
        self.ok(unsafe { ffi::moe_st_load_model(self.st, m.m) })
    }
}

impl Drop for Weights {
    fn drop(&mut self) {
        unsafe { ffi::moe_st_close(self.st) }
    }
}

/// placement.json (main.rs:455): the expert ids of (layer, tier) in slot order.
pub fn placement(path: &str, layer: usize, tier: usize) -> Result<Vec<i32>, Error> {
    let c = std::ffi::CString::new(path).map_err(|_| Error { code: -1, msg: "NUL in path".into() })?;
    let mut n: c_int = 0;
    let err = || cstr(unsafe { ffi::moe_st_last_error(std::ptr::null()) });
    check(unsafe { ffi::moe_placement_read(c.as_ptr(), layer as c_int, tier as c_int, std::ptr::null_mut(), 0, &mut n) }, err)?;
    let mut ids = vec![0i32; n as usize];
    check(unsafe { ffi::moe_placement_read(c.as_ptr(), layer as c_int, tier as c_int, ids.as_mut_ptr(), n, &mut n) }, err)?;
    Ok(ids)
}

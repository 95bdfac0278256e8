//! HIP backend for the Laya decision model: the transformer forward behind
//! `laya_core::Backend` (runtime/crates/laya-core/src/backend.rs:109-133) on an AMD Instinct
//! MI355X (gfx950), through the C ABI of libsys1hip (include/sys1hip.h).
//!
//! It takes laya-mlx's place with the same surface (runtime/crates/laya-mlx/src/lib.rs):
//! `make_backend` has the `BackendFactory` signature (laya-core/src/agent.rs:28-30), `factory`
//! feeds `laya_core::testing::run_parity`, `check_settings` checks a settings string without a
//! model, and `HIP_ENV_DEFAULTS` / `set_hip_env_defaults` stand where `MLX_ENV_DEFAULTS` /
//! `set_mlx_env_defaults` stand. Everything above the trait (tokenizer, collation, decoding, the
//! action head, the server) stays as it is.

mod ffi;

use ffi::*;
use laya_core::{
    Backend, BackendOptions, BackendOutput, Batch, Device, Error, ModelConfig, Result, Weights,
};
use safetensors::Dtype;
use std::ffi::{c_int, CStr, CString};
use std::sync::Mutex;

/// Environment variables this backend sets for itself before its first GPU call, as laya-mlx's
/// `MLX_ENV_DEFAULTS` (lib.rs:278). libsys1hip reads no environment variable, so the list is
/// empty; it exists so that sys1rust and sys1-bench change one crate name and nothing else.
pub const HIP_ENV_DEFAULTS: [(&str, &str); 0] = [];

/// laya-mlx's `set_mlx_env_defaults` (lib.rs:291-297): there is nothing to set, so it returns
/// the empty list of variables it set.
pub fn set_hip_env_defaults() -> Vec<(&'static str, &'static str)> {
    Vec::new()
}

fn error_of(code: c_int) -> Error {
    // SAFETY: s1_last_error returns this thread's NUL-terminated message, valid until the next
    // failing call on the thread.
    let msg = unsafe { CStr::from_ptr(s1_last_error()) }
        .to_string_lossy()
        .into_owned();
    match code {
        S1_ERR_CONFIG => Error::Config(msg),
        S1_ERR_WEIGHTS => Error::Weights(msg),
        _ => Error::Backend(msg), // S1_ERR_BACKEND, and S1_ERR_BATCH for a malformed batch
    }
}

fn check(code: c_int) -> Result<()> {
    if code == S1_OK {
        Ok(())
    } else {
        Err(error_of(code))
    }
}

fn c_string(s: String, what: &str) -> Result<CString> {
    CString::new(s).map_err(|_| Error::Config(format!("{what} contains a NUL byte")))
}

/// laya-mlx's `check_settings` (lib.rs:264-266): the error `make_backend` would return for this
/// settings string, without loading a model. Every key of laya-mlx's `Knobs` is accepted with
/// its value checks (keys that only steer MLX are accepted and do nothing), so sys1rust's
/// `DEFAULT_TUNING` (sys1rust/src/config.rs:29) passes.
pub fn check_settings(spec: &str) -> Result<()> {
    let s = c_string(spec.to_string(), "settings")?;
    check(unsafe { s1_check_settings(s.as_ptr()) })
}

/// The settings libsys1hip gets. laya-mlx keeps the checkpoint's f16 weights unless
/// `BackendOptions::f32` (backend.rs:25-27): `dtype=f16` is that choice here (weights and
/// activations in f16, f32 accumulation), put before the caller's settings so that a `dtype=` of
/// theirs wins (last mention wins; the library's own default is bf16). With `f32` the
/// transformer runs in f32 (`dtype=f32`, after the caller's settings: the option wins, as it
/// does in laya-mlx).
fn library_settings(spec: &str, f32: bool) -> String {
    match (spec.is_empty(), f32) {
        (true, false) => "dtype=f16".to_string(),
        (false, false) => format!("dtype=f16,{spec}"),
        (true, true) => "dtype=f32".to_string(),
        (false, true) => format!("{spec},dtype=f32"),
    }
}

/// `encoder/config.json` as the library reads it, rebuilt from the parsed config (the layer
/// pattern travels as `layer_types`, so a checkpoint's explicit list survives).
fn encoder_json(cfg: &ModelConfig) -> String {
    let e = &cfg.encoder;
    let types: Vec<&str> = e
        .layer_is_local
        .iter()
        .map(|&local| if local { "sliding_attention" } else { "full_attention" })
        .collect();
    serde_json::json!({
        "model_type": "modernbert",
        "vocab_size": e.vocab_size,
        "hidden_size": e.hidden_size,
        "num_hidden_layers": e.num_hidden_layers,
        "num_attention_heads": e.num_attention_heads,
        "intermediate_size": e.intermediate_size,
        "norm_eps": e.norm_eps,
        "global_attn_every_n_layers": e.global_attn_every_n_layers,
        "local_attention": e.local_attention,
        "global_rope_theta": e.global_rope_theta,
        "local_rope_theta": e.local_rope_theta,
        "pad_token_id": e.pad_token_id,
        "max_position_embeddings": e.max_position_embeddings,
        "layer_types": types,
    })
    .to_string()
}

fn agent_json(cfg: &ModelConfig) -> String {
    serde_json::json!({
        "head_layers": cfg.agent.head_layers,
        "max_len": cfg.agent.max_len,
        "head_max_len": cfg.agent.head_max_len,
    })
    .to_string()
}

/// The library's element type code for a safetensors dtype; -1 (refused by the library with a
/// Weights error naming the tensor) for dtypes a Laya checkpoint never holds.
fn dtype_code(d: Dtype) -> i32 {
    match d {
        Dtype::F32 => S1_DTYPE_F32,
        Dtype::F16 => S1_DTYPE_F16,
        Dtype::BF16 => S1_DTYPE_BF16,
        Dtype::F64 => S1_DTYPE_F64,
        _ => -1,
    }
}

pub struct HipBackend {
    model: *mut S1Model,
    hidden: usize,
    kernels: &'static [&'static str],
    /// libsys1hip allows one call at a time per model: its staging buffers and graphs are the
    /// model's. The runtime drives a backend from one inference thread, so the lock is never
    /// contended there; it keeps other callers correct.
    lock: Mutex<()>,
}

// SAFETY: the model handle is only used under `lock` (or in drop, with no other reference).
unsafe impl Send for HipBackend {}
unsafe impl Sync for HipBackend {}

impl Drop for HipBackend {
    fn drop(&mut self) {
        unsafe { s1_model_destroy(self.model) }
    }
}

impl HipBackend {
    /// Load the checkpoint's tensors onto the GPU. `Weights::view` (laya-core/src/weights.rs:46-48)
    /// parses the mapping into (name, dtype, shape, bytes) views; the library copies from them
    /// during the call and keeps no pointer into the mapping.
    pub fn new(w: &Weights, cfg: &ModelConfig, opts: &BackendOptions) -> Result<Self> {
        if opts.device == Device::Cpu {
            return Err(Error::Config(
                "laya-hip runs on an AMD GPU only; Device::Cpu is not supported by this backend"
                    .into(),
            ));
        }
        let settings = c_string(library_settings(&opts.settings(), opts.f32), "settings")?;
        let enc = c_string(encoder_json(cfg), "encoder config")?;
        let agent = c_string(agent_json(cfg), "agent config")?;

        let st = w.view()?;
        let views = st.tensors();
        let names = views
            .iter()
            .map(|(n, _)| c_string(n.clone(), "tensor name"))
            .collect::<Result<Vec<CString>>>()?;
        let shapes: Vec<Vec<u64>> = views
            .iter()
            .map(|(_, v)| v.shape().iter().map(|&s| s as u64).collect())
            .collect();
        let tensors: Vec<S1Tensor> = views
            .iter()
            .zip(names.iter().zip(shapes.iter()))
            .map(|((_, v), (name, shape))| S1Tensor {
                name: name.as_ptr(),
                dtype: dtype_code(v.dtype()),
                ndim: shape.len() as u32,
                shape: shape.as_ptr(),
                data: v.data().as_ptr().cast(),
                nbytes: v.data().len(),
            })
            .collect();

        // Device::Auto and Device::Gpu both mean the first GPU the process sees
        // (HIP_VISIBLE_DEVICES picks which one that is).
        let mut model = std::ptr::null_mut();
        check(unsafe {
            s1_model_create_from_tensors(
                tensors.as_ptr(),
                tensors.len(),
                enc.as_ptr(),
                agent.as_ptr(),
                settings.as_ptr(),
                0,
                &mut model,
            )
        })?;
        // The list is fixed at load; the trait hands out 'static slices, so it is leaked once
        // per model (a few bytes).
        let list = unsafe { CStr::from_ptr(s1_active_kernels(model)) }
            .to_string_lossy()
            .into_owned();
        let kernels: Vec<&'static str> = list
            .split(',')
            .filter(|k| !k.is_empty())
            .map(|k| &*Box::leak(k.to_string().into_boxed_str()))
            .collect();
        Ok(Self {
            model,
            hidden: cfg.hidden_size(),
            kernels: Box::leak(kernels.into_boxed_slice()),
            lock: Mutex::new(()),
        })
    }
}

/// The widths the C ABI takes for a batch's `usize` vectors.
struct Wide {
    seq_lens: Vec<u64>,
    marker_count: Vec<u64>,
}

impl Wide {
    fn of(b: &Batch) -> Self {
        Self {
            seq_lens: b.seq_lens.iter().map(|&x| x as u64).collect(),
            marker_count: b.marker_count.iter().map(|&x| x as u64).collect(),
        }
    }
}

fn dims(b: &Batch) -> Result<(u32, u32, u32)> {
    let fit = |x: usize, what: &str| {
        u32::try_from(x).map_err(|_| Error::Backend(format!("batch {what} {x} does not fit u32")))
    };
    Ok((fit(b.n, "rows")?, fit(b.len, "length")?, fit(b.kmax, "kmax")?))
}

impl Backend for HipBackend {
    fn name(&self) -> String {
        unsafe { CStr::from_ptr(s1_name(self.model)) }
            .to_string_lossy()
            .into_owned()
    }

    fn forward(&self, b: &Batch) -> Result<BackendOutput> {
        let (n, len, kmax) = dims(b)?;
        let wide = Wide::of(b);
        let mut logits = vec![0f32; b.n * b.kmax];
        let mut pooled = vec![0f32; b.n * self.hidden];
        let _g = self.lock.lock().unwrap_or_else(|p| p.into_inner());
        check(unsafe {
            s1_forward(
                self.model,
                n,
                len,
                kmax,
                b.input_ids.as_ptr(),
                b.attention_mask.as_ptr(),
                wide.seq_lens.as_ptr(),
                b.marker_pos.as_ptr(),
                wide.marker_count.as_ptr(),
                b.qtype.as_ptr(),
                logits.as_mut_ptr(),
                pooled.as_mut_ptr(),
            )
        })?;
        Ok(BackendOutput { logits, pooled })
    }

    fn active_kernels(&self) -> &'static [&'static str] {
        self.kernels
    }

    fn padded_len(&self, len: usize, rows: usize) -> usize {
        unsafe { s1_padded_len(self.model, len, rows) }
    }

    fn warmup(&self) -> Result<()> {
        let _g = self.lock.lock().unwrap_or_else(|p| p.into_inner());
        check(unsafe { s1_warmup(self.model) })
    }

    fn encoder_hidden(&self, b: &Batch) -> Result<Option<Vec<f32>>> {
        let (n, len, kmax) = dims(b)?;
        let wide = Wide::of(b);
        let mut hidden = vec![0f32; b.n * b.len * self.hidden];
        let _g = self.lock.lock().unwrap_or_else(|p| p.into_inner());
        check(unsafe {
            s1_encoder_hidden(
                self.model,
                n,
                len,
                kmax,
                b.input_ids.as_ptr(),
                b.attention_mask.as_ptr(),
                wide.seq_lens.as_ptr(),
                b.marker_pos.as_ptr(),
                wide.marker_count.as_ptr(),
                b.qtype.as_ptr(),
                hidden.as_mut_ptr(),
            )
        })?;
        Ok(Some(hidden))
    }
}

/// The `BackendFactory` (laya-core/src/agent.rs:28-30) for `Agent::load`.
pub fn make_backend(
    w: &Weights,
    cfg: &ModelConfig,
    opts: &BackendOptions,
) -> Result<Box<dyn Backend>> {
    Ok(Box::new(HipBackend::new(w, cfg, opts)?))
}

/// Factory for `laya_core::testing::run_parity` (laya-core/src/testing.rs:390-395).
pub fn factory() -> laya_core::testing::Factory {
    Box::new(make_backend)
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn dtype_f16_comes_first_so_the_callers_dtype_wins() {
        assert_eq!(library_settings("", false), "dtype=f16");
        assert_eq!(library_settings("headprune", false), "dtype=f16,headprune");
        assert_eq!(library_settings("dtype=bf16", false), "dtype=f16,dtype=bf16");
    }

    #[test]
    fn the_f32_option_comes_last_so_it_wins() {
        assert_eq!(library_settings("", true), "dtype=f32");
        assert_eq!(library_settings("headprune,dtype=bf16", true), "headprune,dtype=bf16,dtype=f32");
    }

    #[test]
    fn check_settings_matches_laya_mlx_on_the_production_string() {
        check_settings("f16gelu,cache=512,wired=2048,dense_upto=1024,headprune,unpad,fuserope,band=512,nax=all,directload,sharehead,parallel_load").unwrap();
        let e = check_settings("nosuchkey").unwrap_err();
        assert!(matches!(e, Error::Config(ref m) if m.contains("nosuchkey")), "{e}");
    }

    #[test]
    fn device_cpu_is_a_config_error() {
        // Checked before any weight is touched, so no checkpoint is needed: an empty
        // safetensors image (8-byte header length + "{}") stands in.
        let dir = std::env::temp_dir().join(format!("laya-hip-test-{}", std::process::id()));
        std::fs::create_dir_all(&dir).unwrap();
        let mut img = 2u64.to_le_bytes().to_vec();
        img.extend_from_slice(b"{}");
        std::fs::write(dir.join("model.safetensors"), img).unwrap();
        let w = Weights::open(&dir).unwrap();
        let enc = serde_json::json!({
            "model_type": "modernbert", "vocab_size": 64, "hidden_size": 128,
            "num_hidden_layers": 1, "num_attention_heads": 2, "intermediate_size": 64,
        });
        let cfg = ModelConfig {
            agent: serde_json::from_value(serde_json::json!({"encoder": "x"})).unwrap(),
            encoder: laya_core::EncoderConfig::from_value(&enc).unwrap(),
        };
        let opts = BackendOptions { device: Device::Cpu, ..Default::default() };
        let e = HipBackend::new(&w, &cfg, &opts).err().unwrap();
        assert!(matches!(e, Error::Config(_)), "{e}");
        std::fs::remove_dir_all(&dir).ok();
    }
}

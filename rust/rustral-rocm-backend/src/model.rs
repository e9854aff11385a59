//! The config-0 model and the serving step on the device, over the decoder
//! and engine entry points of include/rustral_model.h.
//!
//! * [`RocmDecoder`] stands in for `TransformerDecoder::generate_token`
//!   (crates/nn/src/transformer.rs:837-862): the reference re-runs the whole
//!   prefix through `forward` for every token; here the prefix's K/V rows
//!   stay in paged pools and each new token is one decode step (embedding,
//!   pre-LN layers with paged decode attention, final LN, lm_head, greedy
//!   argmax), replayed from a HIP graph.
//! * [`RocmServingEngine`] stands in for `ServingEngine`
//!   (crates/nn/src/continuous_batching.rs:493-545): `submit`, `step`,
//!   `run_to_completion`; where the reference's step emits a dummy token
//!   (:516-524), this one runs the decoder over the scheduler's batch.

use std::ffi::CString;

use rustral_core::{CoreError, Result};

use crate::error::{check, last_error};
use crate::ffi;
use crate::RocmBackend;

/// Shape of the pre-LN decoder (`rkv_decoder_config`).
#[derive(Clone, Copy, Debug, PartialEq)]
pub struct DecoderConfig {
    pub vocab: usize,
    pub d_model: usize,
    pub n_heads: usize,
    pub n_kv_heads: usize,
    pub d_ff: usize,
    pub n_layers: usize,
    pub max_seq: usize,
    pub eps: f32,
}

impl DecoderConfig {
    /// Benchmark configs[0]: 2 layers, d_model 128, 4 heads of 32, MLP 512,
    /// vocab 1000, pools for 128 positions (a 32-token prompt and 64 new tokens
    /// use 95).
    pub fn config0() -> Self {
        Self { vocab: 1000, d_model: 128, n_heads: 4, n_kv_heads: 4, d_ff: 512, n_layers: 2, max_seq: 128, eps: 1e-5 }
    }

    fn raw(&self) -> Result<ffi::RkvDecoderConfig> {
        let c = |v: usize, what: &str| {
            i32::try_from(v).map_err(|_| CoreError::InvalidArgument(format!("{what} = {v} exceeds i32")))
        };
        Ok(ffi::RkvDecoderConfig {
            vocab: c(self.vocab, "vocab")?,
            d_model: c(self.d_model, "d_model")?,
            n_heads: c(self.n_heads, "n_heads")?,
            n_kv_heads: c(self.n_kv_heads, "n_kv_heads")?,
            d_ff: c(self.d_ff, "d_ff")?,
            n_layers: c(self.n_layers, "n_layers")?,
            max_seq: c(self.max_seq, "max_seq")?,
            eps: self.eps,
        })
    }

    /// Floats in the parameter array (the order of include/rustral_model.h).
    pub fn param_count(&self) -> Result<usize> {
        let raw = self.raw()?;
        // SAFETY: pointer to a live config.
        let n = unsafe { ffi::rkv_decoder_param_count(&raw) };
        usize::try_from(n).map_err(|_| CoreError::InvalidArgument(format!("invalid decoder config {:?}", self)))
    }

    /// The seeded initialisation: weight matrices and the embedding
    /// N(0, std^2) from one PCG64 stream in parameter order, layer-norm gains
    /// 1, biases 0.
    pub fn init_params(&self, seed: u64, std: f32) -> Result<Vec<f32>> {
        let raw = self.raw()?;
        let mut p = vec![0f32; self.param_count()?];
        // SAFETY: p holds param_count floats.
        check(unsafe { ffi::rkv_decoder_init_params(&raw, seed, std, p.as_mut_ptr()) })?;
        Ok(p)
    }
}

fn token_ids(prompt: &[u32], vocab: usize) -> Result<Vec<i32>> {
    prompt
        .iter()
        .map(|&t| {
            if (t as usize) < vocab {
                Ok(t as i32)
            } else {
                Err(CoreError::InvalidArgument(format!("token id {t} outside the vocabulary of {vocab}")))
            }
        })
        .collect()
}

/// The greedy decoder on the device.
pub struct RocmDecoder {
    h: *mut ffi::RkvDecoder,
    cfg: DecoderConfig,
    // keeps the stream the decoder enqueues on alive
    _backend: RocmBackend,
}

// SAFETY: the handle is used through &mut self only.
unsafe impl Send for RocmDecoder {}

impl RocmDecoder {
    /// Uploads `params` (`cfg.param_count()` floats) and allocates the paged
    /// pools, on the backend's stream.
    pub fn new(backend: &RocmBackend, cfg: DecoderConfig, params: &[f32]) -> Result<Self> {
        let raw = cfg.raw()?;
        if params.len() != cfg.param_count()? {
            return Err(CoreError::ShapeMismatch { expected: vec![cfg.param_count()?], actual: vec![params.len()] });
        }
        // SAFETY: params holds n_params floats; the stream outlives the decoder.
        let h = unsafe { ffi::rkv_decoder_create(&raw, params.as_ptr(), params.len() as i64, backend.ctx.stream) };
        if h.is_null() {
            return Err(CoreError::Backend(last_error()));
        }
        Ok(Self { h, cfg, _backend: backend.clone() })
    }

    /// A decoder with `DecoderConfig::init_params(seed, std)` weights.
    pub fn random(backend: &RocmBackend, cfg: DecoderConfig, seed: u64, std: f32) -> Result<Self> {
        Self::new(backend, cfg, &cfg.init_params(seed, std)?)
    }

    /// A decoder whose parameters come from a safetensors file under the
    /// reference's strict `load_model` rules (crates/runtime/src/
    /// model_io.rs:36-105), read straight into device memory.
    pub fn from_safetensors(backend: &RocmBackend, cfg: DecoderConfig, path: &str) -> Result<Self> {
        let raw = cfg.raw()?;
        let cpath = CString::new(path).map_err(|e| CoreError::InvalidArgument(e.to_string()))?;
        // SAFETY: NUL-terminated path; the stream outlives the decoder.
        let h = unsafe { ffi::rkv_decoder_create_from_safetensors(&raw, cpath.as_ptr(), backend.ctx.stream) };
        if h.is_null() {
            return Err(CoreError::Serialization(last_error()));
        }
        Ok(Self { h, cfg, _backend: backend.clone() })
    }

    pub fn config(&self) -> &DecoderConfig {
        &self.cfg
    }

    fn run(&mut self, prompt: &[u32], n_new: usize, logits: Option<&mut Vec<f32>>) -> Result<Vec<u32>> {
        if prompt.is_empty() || n_new == 0 {
            return Err(CoreError::InvalidArgument("generate: an empty prompt or no tokens to generate".into()));
        }
        if prompt.len() + n_new - 1 > self.cfg.max_seq {
            return Err(CoreError::Shape(format!(
                "generate: {} prompt + {n_new} new tokens exceed max_seq {}", prompt.len(), self.cfg.max_seq
            )));
        }
        let ids = token_ids(prompt, self.cfg.vocab)?;
        let mut out = vec![0i32; n_new];
        let lp = match logits {
            Some(v) => {
                v.resize(n_new * self.cfg.vocab, 0.0);
                v.as_mut_ptr()
            }
            None => std::ptr::null_mut(),
        };
        // SAFETY: ids holds n_prompt ids, out n_new, logits NULL or n_new * vocab.
        check(unsafe {
            ffi::rkv_decoder_generate(self.h, ids.as_ptr(), ids.len() as i32, n_new as i32, out.as_mut_ptr(), lp)
        })?;
        Ok(out.into_iter().map(|t| t as u32).collect())
    }

    /// Greedy generation of `n_new` tokens after `prompt`.
    pub fn generate(&mut self, prompt: &[u32], n_new: usize) -> Result<Vec<u32>> {
        self.run(prompt, n_new, None)
    }

    /// `generate` plus each step's logits (`[n_new][vocab]`).
    pub fn generate_with_logits(&mut self, prompt: &[u32], n_new: usize) -> Result<(Vec<u32>, Vec<f32>)> {
        let mut logits = Vec::new();
        let toks = self.run(prompt, n_new, Some(&mut logits))?;
        Ok((toks, logits))
    }

    /// `TransformerDecoder::generate_token` (crates/nn/src/transformer.rs:
    /// 837-862): the greedy next token after `prefix` (the last maximum on
    /// ties, as `max_by` picks it).
    pub fn generate_token(&mut self, prefix: &[usize]) -> Result<u32> {
        let ids: Vec<u32> = prefix
            .iter()
            .map(|&t| u32::try_from(t).map_err(|_| CoreError::InvalidArgument(format!("token id {t}"))))
            .collect::<Result<_>>()?;
        Ok(self.run(&ids, 1, None)?[0])
    }
}

impl Drop for RocmDecoder {
    fn drop(&mut self) {
        // SAFETY: created by rkv_decoder_create*, destroyed once.
        unsafe { ffi::rkv_decoder_destroy(self.h) }
    }
}

/// `RequestPriority` (crates/nn/src/continuous_batching.rs:8-14).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Priority {
    Low,
    Normal,
    High,
    Critical,
}

impl Priority {
    fn code(self) -> i32 {
        match self {
            Priority::Low => ffi::RKV_PRIORITY_LOW,
            Priority::Normal => ffi::RKV_PRIORITY_NORMAL,
            Priority::High => ffi::RKV_PRIORITY_HIGH,
            Priority::Critical => ffi::RKV_PRIORITY_CRITICAL,
        }
    }
}

/// Counts of the engine's scheduler (`Scheduler::stats`,
/// continuous_batching.rs:391-438).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct SchedulerStats {
    pub pending: usize,
    pub running: usize,
    pub paused: usize,
    pub completed: usize,
    pub total_tokens_generated: usize,
}

/// Continuous batching over the decoder: the scheduler's block manager owns
/// `num_blocks` 16-token blocks per layer; each step runs every scheduled
/// request's input rows (a prompt in prefill, the last token otherwise)
/// through the layers with one paged prefill-attention call per layer and
/// hands one greedy token per request back to the scheduler.
pub struct RocmServingEngine {
    h: *mut ffi::RkvEngine,
    cfg: DecoderConfig,
    _backend: RocmBackend,
}

// SAFETY: the handle is used through &mut self only (or read through &self).
unsafe impl Send for RocmServingEngine {}

impl RocmServingEngine {
    pub fn new(backend: &RocmBackend, cfg: DecoderConfig, params: &[f32], num_blocks: usize,
               max_batch_size: usize) -> Result<Self> {
        let raw = cfg.raw()?;
        if params.len() != cfg.param_count()? {
            return Err(CoreError::ShapeMismatch { expected: vec![cfg.param_count()?], actual: vec![params.len()] });
        }
        let mb = i32::try_from(max_batch_size)
            .map_err(|_| CoreError::InvalidArgument(format!("max_batch_size = {max_batch_size} exceeds i32")))?;
        // SAFETY: params holds n_params floats; the stream outlives the engine.
        let h = unsafe {
            ffi::rkv_engine_create(&raw, params.as_ptr(), params.len() as i64, num_blocks as i64, mb,
                                   backend.ctx.stream)
        };
        if h.is_null() {
            return Err(CoreError::Backend(last_error()));
        }
        Ok(Self { h, cfg, _backend: backend.clone() })
    }

    /// `ServingEngine::submit` (continuous_batching.rs:507-510): queues a
    /// request at normal priority and returns its id.
    pub fn submit(&mut self, prompt: Vec<u32>, max_tokens: usize) -> Result<u64> {
        self.submit_with_priority(&prompt, max_tokens, Priority::Normal)
    }

    /// `Scheduler::add_priority_request` (:230-246) through the engine.
    pub fn submit_with_priority(&mut self, prompt: &[u32], max_tokens: usize, priority: Priority) -> Result<u64> {
        let ids = token_ids(prompt, self.cfg.vocab)?;
        let mt = i32::try_from(max_tokens)
            .map_err(|_| CoreError::InvalidArgument(format!("max_tokens = {max_tokens} exceeds i32")))?;
        // SAFETY: ids holds n_prompt ids.
        let id = unsafe { ffi::rkv_engine_submit(self.h, ids.as_ptr(), ids.len() as i32, mt, priority.code()) };
        if id < 0 {
            check(id as i32)?;
        }
        Ok(id as u64)
    }

    /// `ServingEngine::step` (:513-535): one scheduled batch through the
    /// model; returns how many requests ran (0: nothing was scheduled).  An
    /// exhausted pool is `CoreError::Other`, as `Scheduler::update` reports it.
    pub fn step(&mut self) -> Result<usize> {
        // SAFETY: valid handle.
        let rc = unsafe { ffi::rkv_engine_step(self.h) };
        check(rc.min(0))?;
        Ok(rc as usize)
    }

    /// `ServingEngine::run_to_completion` (:538-543): steps until no request
    /// is pending, running or paused; returns the number of steps.
    pub fn run_to_completion(&mut self) -> Result<usize> {
        // SAFETY: valid handle.
        let rc = unsafe { ffi::rkv_engine_run(self.h, i32::MAX) };
        check(rc.min(0))?;
        Ok(rc as usize)
    }

    /// The tokens a request has generated so far (running, paused or
    /// completed).
    pub fn generated(&self, request_id: u64) -> Result<Vec<u32>> {
        // SAFETY: the scheduler is owned by the engine; a NULL buffer asks for the count.
        unsafe {
            let s = ffi::rkv_engine_scheduler(self.h);
            let n = ffi::rkv_sched_generated(s, request_id as i64, std::ptr::null_mut(), 0);
            if n < 0 {
                check(n as i32)?;
            }
            let mut v = vec![0i32; n as usize];
            ffi::rkv_sched_generated(s, request_id as i64, v.as_mut_ptr(), n);
            Ok(v.into_iter().map(|t| t as u32).collect())
        }
    }

    pub fn stats(&self) -> Result<SchedulerStats> {
        let mut o = [0i64; 5];
        // SAFETY: the scheduler is owned by the engine; o holds 5 entries.
        check(unsafe { ffi::rkv_sched_stats(ffi::rkv_engine_scheduler(self.h), o.as_mut_ptr()) })?;
        Ok(SchedulerStats {
            pending: o[0] as usize,
            running: o[1] as usize,
            paused: o[2] as usize,
            completed: o[3] as usize,
            total_tokens_generated: o[4] as usize,
        })
    }

    /// `Scheduler::is_empty`: nothing pending, running or paused.
    pub fn is_empty(&self) -> Result<bool> {
        let s = self.stats()?;
        Ok(s.pending + s.running + s.paused == 0)
    }
}

impl Drop for RocmServingEngine {
    fn drop(&mut self) {
        // SAFETY: created by rkv_engine_create, destroyed once.
        unsafe { ffi::rkv_engine_destroy(self.h) }
    }
}

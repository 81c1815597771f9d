//! `turboquant_cache::KVCache` (crates/turboquant-cache/src/traits.rs:9-36)
//! over libtqkv's device cache (`tqkv_kvcache_*`): a drop-in for
//! `SimpleCache` (crates/turboquant-cache/src/simple.rs:13-149) whose
//! compressed vectors live on the GPU. Given the same R and Phi, the stored
//! codes (packed as `CompressedVector::stage1_packed`), scales, QJL signs and
//! residual norms equal `TurboQuantCompressor::compress`'s, and
//! `attend_keys` / `attend_values` return `SimpleCache`'s results bit for
//! bit.
//!
//! Calls are synchronous and take host slices, as the trait does. The
//! library stages inputs through a device buffer owned by the cache, so
//! every call, `&self` ones included, holds the cache's lock: the type is
//! `Send + Sync` through that lock, as the trait requires.
//!
//! The trait methods panic where `SimpleCache` panics (a layer or head out
//! of range, slices of the wrong length) and on a device error, with the
//! library's message. The `try_*` methods return the error instead.

use std::ffi::CStr;
use std::fmt;
use std::ptr::{self, NonNull};
use std::sync::{Mutex, MutexGuard};

use tqkv_sys as sys;
use turboquant_cache::traits::KVCache;

/// A libtqkv status other than `TQKV_OK`, with the library's message.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct Error {
    pub status: i32,
    pub message: String,
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "libtqkv status {}: {}", self.status, self.message)
    }
}

impl std::error::Error for Error {}

fn error(status: i32, message: String) -> Error {
    Error { status, message }
}

fn check(status: i32) -> Result<(), Error> {
    if status == sys::TQKV_OK {
        return Ok(());
    }
    // SAFETY: tqkv_last_error returns null or this thread's NUL-terminated
    // message, valid until the next library call on this thread; it is
    // copied out before any other call.
    let message = unsafe {
        let p = sys::tqkv_last_error();
        if p.is_null() {
            String::new()
        } else {
            CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    };
    Err(error(status, message))
}

fn narrow(v: usize, what: &str) -> Result<i32, Error> {
    i32::try_from(v).map_err(|_| error(sys::TQKV_EINVAL_ARG, format!("{what}={v} out of range")))
}

/// `TurboQuantConfig` (crates/lumen-core/src/config.rs:5-28).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub struct Config {
    pub head_dim: usize,
    pub bits: u32,
    pub qjl_m: usize,
    /// Lloyd-Max iterations; 0 means the reference's 1000.
    pub lloyd_max_iter: usize,
    pub seed: u64,
}

impl Config {
    fn raw(&self) -> Result<sys::tqkv_tq_config, Error> {
        Ok(sys::tqkv_tq_config {
            head_dim: narrow(self.head_dim, "head_dim")?,
            bits: narrow(self.bits as usize, "bits")?,
            qjl_m: narrow(self.qjl_m, "qjl_m")?,
            lloyd_max_iter: narrow(self.lloyd_max_iter, "lloyd_max_iter")?,
            seed: self.seed,
        })
    }
}

/// The stored fields of a run of compressed vectors: codes unpacked to one
/// byte each ([n, head_dim]), scales, QJL sign words ([n, ceil(qjl_m / 32)])
/// and residual norms.
#[derive(Debug, Clone, PartialEq)]
pub struct Stored {
    pub codes: Vec<u8>,
    pub scale: Vec<f32>,
    pub signs: Vec<u32>,
    pub residual_norm: Vec<f32>,
}

struct Raw(NonNull<sys::tqkv_kvcache>);

// SAFETY: the library's cache object has no thread affinity (any host thread
// may call it); DeviceCache serializes every call through its Mutex.
unsafe impl Send for Raw {}

/// The device cache. Dropping it frees its device memory.
pub struct DeviceCache {
    raw: Mutex<Raw>,
    n_layers: usize,
    n_kv_heads: usize,
    head_dim: usize,
    qjl_m: usize,
}

impl DeviceCache {
    /// `SimpleCache::new` over `TurboQuantCompressor::new(config)`
    /// (compressor.rs:20-32): R drawn at `seed`, Phi at `seed + 1`.
    pub fn new(config: &Config, n_layers: usize, n_kv_heads: usize) -> Result<Self, Error> {
        Self::create(config, None, None, n_layers, n_kv_heads)
    }

    /// `SimpleCache::new` over `TurboQuantCompressor::from_files`
    /// (compressor.rs:35-58): R row-major [head_dim, head_dim] and Phi
    /// [qjl_m, head_dim] as given.
    pub fn with_tables(
        config: &Config,
        rotation: &[f32],
        qjl: &[f32],
        n_layers: usize,
        n_kv_heads: usize,
    ) -> Result<Self, Error> {
        let d = config.head_dim;
        if Some(rotation.len()) != d.checked_mul(d) || Some(qjl.len()) != config.qjl_m.checked_mul(d)
        {
            return Err(error(
                sys::TQKV_EINVAL_SHAPE,
                format!(
                    "rotation has {} floats and qjl {}, want {d}x{d} and {}x{d}",
                    rotation.len(),
                    qjl.len(),
                    config.qjl_m
                ),
            ));
        }
        Self::create(config, Some(rotation), Some(qjl), n_layers, n_kv_heads)
    }

    fn create(
        config: &Config,
        rotation: Option<&[f32]>,
        qjl: Option<&[f32]>,
        n_layers: usize,
        n_kv_heads: usize,
    ) -> Result<Self, Error> {
        let cfg = config.raw()?;
        let layers = narrow(n_layers, "n_layers")?;
        let heads = narrow(n_kv_heads, "n_kv_heads")?;
        let mut out: *mut sys::tqkv_kvcache = ptr::null_mut();
        // SAFETY: cfg outlives the call; rotation and qjl are null or hold
        // the head_dim^2 and qjl_m * head_dim floats the library reads
        // (with_tables checks the lengths); out is a valid place to write.
        check(unsafe {
            sys::tqkv_kvcache_create(
                &cfg,
                rotation.map_or(ptr::null(), <[f32]>::as_ptr),
                qjl.map_or(ptr::null(), <[f32]>::as_ptr),
                layers,
                heads,
                &mut out,
            )
        })?;
        let raw = NonNull::new(out)
            .ok_or_else(|| error(sys::TQKV_EDEVICE, "tqkv_kvcache_create returned null".into()))?;
        Ok(Self {
            raw: Mutex::new(Raw(raw)),
            n_layers,
            n_kv_heads,
            head_dim: config.head_dim,
            qjl_m: config.qjl_m,
        })
    }

    fn lock(&self) -> MutexGuard<'_, Raw> {
        // A panic in another caller cannot leave the library object half
        // updated (each call completes or fails as a whole), so a poisoned
        // lock is still usable.
        self.raw.lock().unwrap_or_else(|e| e.into_inner())
    }

    fn index(&self, layer: usize, head: usize) -> Result<(i32, i32), Error> {
        if layer >= self.n_layers || head >= self.n_kv_heads {
            return Err(error(
                sys::TQKV_EINVAL_ARG,
                format!(
                    "layer {layer} / head {head} out of range ({} x {})",
                    self.n_layers, self.n_kv_heads
                ),
            ));
        }
        Ok((layer as i32, head as i32))
    }

    fn len_locked(raw: &Raw, layer: i32, head: i32) -> usize {
        // SAFETY: raw is a live cache; layer and head were range-checked.
        let n = unsafe { sys::tqkv_kvcache_seq_len(raw.0.as_ptr(), layer, head) };
        usize::try_from(n).unwrap_or(0)
    }

    pub fn head_dim(&self) -> usize {
        self.head_dim
    }

    pub fn try_store(
        &mut self,
        layer: usize,
        head: usize,
        keys: &[f32],
        values: &[f32],
        n_tokens: usize,
    ) -> Result<(), Error> {
        let (l, h) = self.index(layer, head)?;
        let want = n_tokens.checked_mul(self.head_dim);
        if Some(keys.len()) != want || Some(values.len()) != want {
            return Err(error(
                sys::TQKV_EINVAL_SHAPE,
                format!(
                    "{} key and {} value floats for {n_tokens} tokens of {}",
                    keys.len(),
                    values.len(),
                    self.head_dim
                ),
            ));
        }
        let n = i64::try_from(n_tokens)
            .map_err(|_| error(sys::TQKV_EINVAL_SHAPE, format!("n_tokens={n_tokens}")))?;
        let raw = self.lock();
        // SAFETY: keys and values each hold n_tokens * head_dim floats.
        check(unsafe {
            sys::tqkv_kvcache_store(raw.0.as_ptr(), l, h, keys.as_ptr(), values.as_ptr(), n)
        })
    }

    pub fn try_attend_keys(&self, layer: usize, head: usize, query: &[f32]) -> Result<Vec<f32>, Error> {
        let (l, h) = self.index(layer, head)?;
        if query.len() != self.head_dim {
            return Err(error(
                sys::TQKV_EINVAL_SHAPE,
                format!("query of {} floats, head_dim {}", query.len(), self.head_dim),
            ));
        }
        let raw = self.lock();
        let mut scores = vec![0.0f32; Self::len_locked(&raw, l, h)];
        // SAFETY: query holds head_dim floats; scores has room for seq_len
        // floats, taken under the lock every store and truncate also holds.
        check(unsafe {
            sys::tqkv_kvcache_attend_keys(raw.0.as_ptr(), l, h, query.as_ptr(), scores.as_mut_ptr())
        })?;
        Ok(scores)
    }

    pub fn try_attend_values(
        &self,
        layer: usize,
        head: usize,
        weights: &[f32],
    ) -> Result<Vec<f32>, Error> {
        let (l, h) = self.index(layer, head)?;
        let raw = self.lock();
        let n = Self::len_locked(&raw, l, h);
        if weights.len() != n {
            return Err(error(
                sys::TQKV_EINVAL_SHAPE,
                format!("{} weights for {n} cached tokens", weights.len()),
            ));
        }
        let mut out = vec![0.0f32; self.head_dim];
        // SAFETY: weights holds seq_len floats (checked under the lock); out
        // has room for head_dim floats.
        check(unsafe {
            sys::tqkv_kvcache_attend_values(raw.0.as_ptr(), l, h, weights.as_ptr(), out.as_mut_ptr())
        })?;
        Ok(out)
    }

    pub fn try_seq_len(&self, layer: usize, head: usize) -> Result<usize, Error> {
        let (l, h) = self.index(layer, head)?;
        Ok(Self::len_locked(&self.lock(), l, h))
    }

    pub fn try_clear(&mut self) -> Result<(), Error> {
        let raw = self.lock();
        // SAFETY: raw is a live cache.
        check(unsafe { sys::tqkv_kvcache_clear(raw.0.as_ptr()) })
    }

    pub fn try_truncate(&mut self, layer: usize, n_keep: usize) -> Result<(), Error> {
        let (l, _) = self.index(layer, 0)?;
        let keep = i64::try_from(n_keep).unwrap_or(i64::MAX);
        let raw = self.lock();
        // SAFETY: raw is a live cache; layer was range-checked.
        check(unsafe { sys::tqkv_kvcache_truncate(raw.0.as_ptr(), l, keep) })
    }

    /// `SimpleCache::memory_bytes` (simple.rs:65-80): the sum of
    /// `CompressedVector::size_bytes` over the stored vectors.
    pub fn memory_bytes(&self) -> usize {
        let raw = self.lock();
        // SAFETY: raw is a live cache.
        usize::try_from(unsafe { sys::tqkv_kvcache_memory_bytes(raw.0.as_ptr()) }).unwrap_or(0)
    }

    /// Device bytes: (held by the stored vectors, reserved by the cache in
    /// all).
    pub fn device_bytes(&self) -> Result<(usize, usize), Error> {
        let (mut held, mut reserved) = (0i64, 0i64);
        let raw = self.lock();
        // SAFETY: raw is a live cache; both outputs are valid places.
        check(unsafe { sys::tqkv_kvcache_device_bytes(raw.0.as_ptr(), &mut held, &mut reserved) })?;
        Ok((usize::try_from(held).unwrap_or(0), usize::try_from(reserved).unwrap_or(0)))
    }

    /// The stored fields of vectors [first, first + n) of the keys
    /// (`values` false) or values of a (layer, head).
    pub fn read(
        &self,
        layer: usize,
        head: usize,
        values: bool,
        first: usize,
        n: usize,
    ) -> Result<Stored, Error> {
        let (l, h) = self.index(layer, head)?;
        let words = self.qjl_m.div_ceil(32);
        let raw = self.lock();
        let held = Self::len_locked(&raw, l, h);
        if first.checked_add(n).map_or(true, |end| end > held) {
            return Err(error(
                sys::TQKV_EINVAL_TARGET,
                format!("vectors [{first}, {first} + {n}) of {held}"),
            ));
        }
        let mut s = Stored {
            codes: vec![0u8; n * self.head_dim],
            scale: vec![0.0f32; n],
            signs: vec![0u32; n * words],
            residual_norm: vec![0.0f32; if words > 0 { n } else { 0 }],
        };
        let (signs, rnorm) = if words > 0 {
            (s.signs.as_mut_ptr(), s.residual_norm.as_mut_ptr())
        } else {
            (ptr::null_mut(), ptr::null_mut())
        };
        // SAFETY: the range was checked against seq_len under the lock; each
        // output has room for what the library writes for n vectors.
        check(unsafe {
            sys::tqkv_kvcache_read(
                raw.0.as_ptr(),
                l,
                h,
                i32::from(values),
                first as i64,
                n as i64,
                s.codes.as_mut_ptr(),
                s.scale.as_mut_ptr(),
                signs,
                rnorm,
            )
        })?;
        Ok(s)
    }
}

impl Drop for DeviceCache {
    fn drop(&mut self) {
        let raw = self.raw.get_mut().unwrap_or_else(|e| e.into_inner());
        // SAFETY: the pointer came from tqkv_kvcache_create and is destroyed
        // exactly once, here.
        unsafe {
            sys::tqkv_kvcache_destroy(raw.0.as_ptr());
        }
    }
}

impl KVCache for DeviceCache {
    fn store(&mut self, layer: usize, head: usize, keys: &[f32], values: &[f32], n_tokens: usize) {
        if let Err(e) = self.try_store(layer, head, keys, values, n_tokens) {
            panic!("KVCache::store: {e}");
        }
    }

    fn attend_keys(&self, layer: usize, head: usize, query: &[f32]) -> Vec<f32> {
        self.try_attend_keys(layer, head, query)
            .unwrap_or_else(|e| panic!("KVCache::attend_keys: {e}"))
    }

    fn attend_values(&self, layer: usize, head: usize, weights: &[f32]) -> Vec<f32> {
        self.try_attend_values(layer, head, weights)
            .unwrap_or_else(|e| panic!("KVCache::attend_values: {e}"))
    }

    fn seq_len(&self, layer: usize, head: usize) -> usize {
        self.try_seq_len(layer, head).unwrap_or_else(|e| panic!("KVCache::seq_len: {e}"))
    }

    fn clear(&mut self) {
        if let Err(e) = self.try_clear() {
            panic!("KVCache::clear: {e}");
        }
    }

    fn truncate(&mut self, layer: usize, n_keep: usize) {
        if let Err(e) = self.try_truncate(layer, n_keep) {
            panic!("KVCache::truncate: {e}");
        }
    }
}

//! DeviceCache against the reference's SimpleCache, through the KVCache
//! trait, on one GPU: the same R and Phi (taken from the reference's own
//! seeded constructors), the same inputs, and every result compared bit for
//! bit. Needs a gfx950 GPU and libtqkv.so (found as tqkv-sys's build.rs
//! says).

use std::sync::Arc;

use lumen_core::compressor::TurboQuantCompressor;
use lumen_core::config::TurboQuantConfig;
use lumen_core::qjl::QJLProjector;
use tqkv::{Config, DeviceCache};
use turboquant_cache::simple::SimpleCache;
use turboquant_cache::traits::KVCache;

/// Seeded N(0, 1) floats: xorshift64* uniforms through Box-Muller.
fn normals(seed: u64, n: usize) -> Vec<f32> {
    let mut s = seed.wrapping_mul(0x9E37_79B9_7F4A_7C15) | 1;
    let mut uniform = move || {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        (s.wrapping_mul(0x2545_F491_4F6C_DD1D) >> 11) as f64 / (1u64 << 53) as f64
    };
    (0..n)
        .map(|_| {
            let u1 = uniform().max(f64::MIN_POSITIVE);
            let u2 = uniform();
            ((-2.0 * u1.ln()).sqrt() * (std::f64::consts::TAU * u2).cos()) as f32
        })
        .collect()
}

fn bits_of(v: &[f32]) -> Vec<u32> {
    v.iter().map(|x| x.to_bits()).collect()
}

fn pair(dim: usize, bits: u32, m: usize, layers: usize, heads: usize) -> (SimpleCache, DeviceCache) {
    let config = TurboQuantConfig { bits, qjl_m: m, seed: 42, lloyd_max_iter: 1000, head_dim: dim };
    let compressor = Arc::new(TurboQuantCompressor::new(config.clone()));
    let phi = QJLProjector::new(dim, m, config.seed.wrapping_add(1));
    let device = DeviceCache::with_tables(
        &Config { head_dim: dim, bits, qjl_m: m, lloyd_max_iter: 1000, seed: 42 },
        &compressor.rotation().matrix,
        &phi.proj_matrix,
        layers,
        heads,
    )
    .expect("device cache");
    (SimpleCache::new(compressor, layers, heads, dim), device)
}

#[test]
fn scores_and_values_match_simple_cache() {
    for &(dim, bits, m) in &[(64usize, 3u32, 64usize), (128, 4, 64), (128, 2, 32), (256, 3, 128)] {
        let (mut host, mut dev) = pair(dim, bits, m, 2, 3);
        let n = 37;
        let keys = normals(dim as u64 + 1, n * dim);
        let values = normals(dim as u64 + 2, n * dim);
        // Two stores append, as on the reference.
        for cache in [&mut host as &mut dyn KVCache, &mut dev as &mut dyn KVCache] {
            cache.store(1, 2, &keys[..20 * dim], &values[..20 * dim], 20);
            cache.store(1, 2, &keys[20 * dim..], &values[20 * dim..], n - 20);
        }
        assert_eq!(dev.seq_len(1, 2), host.seq_len(1, 2));
        assert_eq!(dev.seq_len(0, 0), 0);
        let q = normals(dim as u64 + 3, dim);
        let s_host = host.attend_keys(1, 2, &q);
        let s_dev = dev.attend_keys(1, 2, &q);
        assert_eq!(bits_of(&s_dev), bits_of(&s_host), "scores dim={dim} bits={bits}");
        let top = s_host.iter().cloned().fold(f32::NEG_INFINITY, f32::max);
        let mut w: Vec<f32> = s_host.iter().map(|s| (s - top).exp()).collect();
        let total: f32 = w.iter().sum();
        w.iter_mut().for_each(|x| *x /= total);
        w[4] = 1e-12; // below the skip threshold on both sides
        assert_eq!(
            bits_of(&dev.attend_values(1, 2, &w)),
            bits_of(&host.attend_values(1, 2, &w)),
            "values dim={dim} bits={bits}"
        );
        assert_eq!(dev.memory_bytes(), host.memory_bytes());
        let (held, reserved) = dev.device_bytes().expect("device bytes");
        assert!(held <= dev.memory_bytes() && reserved >= held);
        for cache in [&mut host as &mut dyn KVCache, &mut dev as &mut dyn KVCache] {
            cache.truncate(1, 11);
        }
        assert_eq!(dev.seq_len(1, 2), 11);
        assert_eq!(bits_of(&dev.attend_keys(1, 2, &q)), bits_of(&host.attend_keys(1, 2, &q)));
        dev.clear();
        assert_eq!(dev.seq_len(1, 2), 0);
        assert_eq!(dev.memory_bytes(), 0);
    }
}

#[test]
fn errors_are_returned_by_try_and_panic_through_the_trait() {
    let (_, mut dev) = pair(64, 3, 64, 1, 1);
    let x = normals(5, 64);
    assert_eq!(dev.try_store(1, 0, &x, &x, 1).unwrap_err().status, tqkv_sys::TQKV_EINVAL_ARG);
    assert_eq!(dev.try_store(0, 0, &x[..63], &x, 1).unwrap_err().status, tqkv_sys::TQKV_EINVAL_SHAPE);
    assert_eq!(dev.try_attend_values(0, 0, &[1.0]).unwrap_err().status, tqkv_sys::TQKV_EINVAL_SHAPE);
    let caught = std::panic::catch_unwind(std::panic::AssertUnwindSafe(|| dev.seq_len(0, 1)));
    assert!(caught.is_err(), "an out-of-range head panics, as SimpleCache's index does");
}

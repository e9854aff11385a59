//! configs[0] end to end on the ROCm backend, run with `cargo test` on an
//! MI355X: the decoder's 64 greedy tokens equal the CPU oracle's
//! (tests/golden/config0_tokens.txt of this repository, written by
//! tests/golden/make_config0_tokens.py), `generate_token` over a growing
//! prefix gives the same tokens one at a time, and the serving engine
//! generates them for the same request.
use rustral_rocm_backend::{DecoderConfig, RocmBackend, RocmDecoder, RocmServingEngine};

/// (prompt, expected tokens) from the fixture; RUSTRAL_AMD_GOLDEN names its
/// directory when the crate is built outside this repository.
fn fixture() -> (Vec<u32>, Vec<u32>) {
    let dir = std::env::var("RUSTRAL_AMD_GOLDEN")
        .unwrap_or_else(|_| format!("{}/../../tests/golden", env!("CARGO_MANIFEST_DIR")));
    let text = std::fs::read_to_string(format!("{dir}/config0_tokens.txt")).expect("config0_tokens.txt");
    let row = |key: &str| -> Vec<u32> {
        let line = text.lines().find(|l| l.starts_with(key)).expect(key);
        line[key.len()..].split_whitespace().map(|t| t.parse().unwrap()).collect()
    };
    (row("prompt "), row("tokens "))
}

#[test]
fn config0_decoder_tokens_equal_the_cpu_path() {
    let gpu = RocmBackend::new(0).expect("a GPU");
    let cfg = DecoderConfig::config0();
    let (prompt, want) = fixture();
    assert_eq!((prompt.len(), want.len()), (32, 64));
    let mut dec = RocmDecoder::random(&gpu, cfg, 0, 0.02).unwrap();
    assert_eq!(dec.generate(&prompt, 64).unwrap(), want);
    // a second call replays the captured launch sequence
    assert_eq!(dec.generate(&prompt, 64).unwrap(), want);
    // generate_token over the growing prefix (TransformerDecoder::generate_token)
    let mut prefix: Vec<usize> = prompt.iter().map(|&t| t as usize).collect();
    for &t in want.iter().take(8) {
        assert_eq!(dec.generate_token(&prefix).unwrap(), t);
        prefix.push(t as usize);
    }
    // out-of-vocabulary ids and an overlong request are errors, not launches
    assert!(dec.generate(&[1000], 1).is_err());
    assert!(dec.generate(&prompt, 200).is_err());
}

#[test]
fn config0_serving_engine_generates_the_same_tokens() {
    let gpu = RocmBackend::new(0).expect("a GPU");
    let cfg = DecoderConfig::config0();
    let (prompt, want) = fixture();
    let params = cfg.init_params(0, 0.02).unwrap();
    let mut eng = RocmServingEngine::new(&gpu, cfg, &params, 64, 4).unwrap();
    let id = eng.submit(prompt.clone(), 64).unwrap();
    let other = eng.submit(prompt[..5].to_vec(), 10).unwrap();
    let steps = eng.run_to_completion().unwrap();
    assert!(steps >= 64);
    assert!(eng.is_empty().unwrap());
    assert_eq!(eng.generated(id).unwrap(), want);
    assert_eq!(eng.generated(other).unwrap().len(), 10);
    let st = eng.stats().unwrap();
    assert_eq!((st.completed, st.total_tokens_generated), (2, 74));
}

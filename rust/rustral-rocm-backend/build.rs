//! Builds librustral_kv for gfx950 from the library sources and links it.
//!
//! Every `*.hip` file of the source directory is compiled with `hipcc` and
//! every `*.cpp` file (host-only code: block manager, scheduler, safetensors
//! reader) with the C++ compiler, with the flags of `rustral_amd/build.py`;
//! the objects are linked into one shared library in OUT_DIR.  No CUDA, no
//! dual code paths: the only target is `--offload-arch=gfx950`.
use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

const ARCH: &str = "gfx950";

fn hipcc() -> PathBuf {
    if let Ok(p) = env::var("HIPCC") {
        return PathBuf::from(p);
    }
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    Path::new(&rocm).join("bin").join("hipcc")
}

fn run(cmd: &mut Command, what: &str) {
    let status = cmd.status().unwrap_or_else(|e| panic!("{what}: cannot start: {e}"));
    assert!(status.success(), "{what} failed ({status})");
}

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    // the crate sits in rustral's crates/rocm-backend; the sources in a
    // checkout of this repository (or a vendored copy of its csrc/ and include/)
    let csrc = env::var("RUSTRAL_AMD_CSRC")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("../../rustral_amd/csrc"));
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let mut sources: Vec<PathBuf> = std::fs::read_dir(&csrc)
        .unwrap_or_else(|e| panic!("cannot read {}: {e}", csrc.display()))
        .filter_map(|e| e.ok().map(|e| e.path()))
        .filter(|p| matches!(p.extension().and_then(|x| x.to_str()), Some("hip") | Some("cpp")))
        .collect();
    sources.sort();
    assert!(!sources.is_empty(), "no .hip / .cpp sources in {}", csrc.display());
    let mut objs = Vec::new();
    for src in &sources {
        let name = src.file_name().unwrap().to_string_lossy().into_owned();
        let obj = out.join(format!("{name}.o"));
        if name.ends_with(".hip") {
            run(
                Command::new(hipcc())
                    .arg(format!("--offload-arch={ARCH}"))
                    .args(["-O3", "-std=c++17", "-fPIC", "-Wall"])
                    // packed fp32 ops stay off (the same flag as rustral_amd/build.py)
                    .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
                    .arg("-c")
                    .arg(src)
                    .arg("-o")
                    .arg(&obj),
                &format!("hipcc {name}"),
            );
        } else {
            let cxx = env::var("CXX").unwrap_or_else(|_| "c++".to_string());
            run(
                Command::new(cxx)
                    .args(["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-c"])
                    .arg(src)
                    .arg("-o")
                    .arg(&obj),
                &format!("c++ {name}"),
            );
        }
        objs.push(obj);
        println!("cargo:rerun-if-changed={}", src.display());
    }
    let lib = out.join("librustral_kv.so");
    run(
        Command::new(hipcc())
            .arg(format!("--offload-arch={ARCH}"))
            .args(["-shared", "-fPIC", "-o"])
            .arg(&lib)
            .args(&objs),
        "link librustral_kv.so",
    );
    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-env-changed=RUSTRAL_AMD_CSRC");
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=rustral_kv");
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
}

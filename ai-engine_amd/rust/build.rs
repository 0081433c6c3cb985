//! build.rs -- Cargo build script of `crates/ai-engine-candle` when its paged
//! engine runs on libpagedkv.  It compiles the library's HIP and C++ sources
//! for gfx950 with hipcc (through the library's own build script, which
//! names every source and flag), then tells rustc where the shared object
//! is.  PAGEDKV_ROOT points at a checkout of the MI355X paged-KV engine.
use std::env;
use std::path::PathBuf;
use std::process::Command;

fn main() {
    // only with the `rocm` feature, beside the crate's cpu|cuda|metal
    // features (crates/ai-engine-candle/Cargo.toml:7-11)
    if env::var_os("CARGO_FEATURE_ROCM").is_none() {
        return;
    }
    let root = PathBuf::from(
        env::var("PAGEDKV_ROOT").expect("PAGEDKV_ROOT: checkout of the MI355X paged-KV engine"),
    );
    let pkg = root.join("ai-engine_amd");
    let python = env::var("PYTHON").unwrap_or_else(|_| "python3".into());
    // hipcc --offload-arch=gfx950 of csrc/*.{hip,cpp} into ai-engine_amd/libpagedkv.so
    let status = Command::new(python)
        .arg(pkg.join("build.py"))
        .status()
        .expect("running ai-engine_amd/build.py");
    assert!(status.success(), "libpagedkv build failed");
    println!("cargo:rustc-link-search=native={}", pkg.display());
    println!("cargo:rustc-link-lib=dylib=pagedkv");
    // the engine finds the library next to the checkout at run time
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", pkg.display());
    println!("cargo:rerun-if-env-changed=PAGEDKV_ROOT");
    println!("cargo:rerun-if-changed={}", pkg.join("csrc").display());
    println!("cargo:rerun-if-changed={}", root.join("include").join("pagedkv.h").display());
}

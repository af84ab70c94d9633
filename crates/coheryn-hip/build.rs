//! Compiles libcohx.so with hipcc for gfx950 into OUT_DIR and links the crate
//! against it.
//!
//! The HIP sources, flags and link line are the ones
//! `coheryn-ai-studio_amd/build.py` uses: both read
//! `coheryn-ai-studio_amd/build.manifest`.  Environment:
//!   COHX_SRC_DIR      folder holding build.manifest and csrc/
//!                     (default: ../../coheryn-ai-studio_amd from this crate)
//!   COHX_INCLUDE_DIR  folder holding cohx.h (default: ../../include)
//!   HIPCC             the compiler (default: /opt/rocm/bin/hipcc)
//!   COHX_ARCH         offload architecture (default: gfx950)
use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

fn manifest(path: &Path) -> Vec<(String, Vec<String>)> {
    let text = std::fs::read_to_string(path)
        .unwrap_or_else(|e| panic!("cannot read {}: {e}", path.display()));
    let mut sections: Vec<(String, Vec<String>)> = Vec::new();
    for raw in text.lines() {
        let line = raw.split('#').next().unwrap_or("").trim();
        if line.is_empty() {
            continue;
        }
        if line.starts_with('[') && line.ends_with(']') {
            sections.push((line[1..line.len() - 1].to_string(), Vec::new()));
        } else if let Some((_, items)) = sections.last_mut() {
            items.push(line.to_string());
        }
    }
    sections
}

fn section<'a>(m: &'a [(String, Vec<String>)], name: &str) -> &'a [String] {
    m.iter()
        .find(|(n, _)| n == name)
        .map(|(_, v)| v.as_slice())
        .unwrap_or_else(|| panic!("build.manifest has no [{name}] section"))
}

fn run(cmd: &mut Command) {
    let status = cmd.status().unwrap_or_else(|e| panic!("cannot run {cmd:?}: {e}"));
    assert!(status.success(), "{cmd:?} failed with {status}");
}

fn main() {
    let crate_dir = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let src_dir = env::var_os("COHX_SRC_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|| crate_dir.join("../../coheryn-ai-studio_amd"));
    let include_dir = env::var_os("COHX_INCLUDE_DIR")
        .map(PathBuf::from)
        .unwrap_or_else(|| crate_dir.join("../../include"));
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".into());
    let arch = env::var("COHX_ARCH").unwrap_or_else(|_| "gfx950".into());
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());

    let m = manifest(&src_dir.join("build.manifest"));
    let flags = section(&m, "flags");
    let mut objects = Vec::new();
    for src in section(&m, "sources") {
        let path = src_dir.join(src);
        let obj = out.join(format!("{}.o", Path::new(src).file_name().unwrap().to_string_lossy()));
        run(Command::new(&hipcc)
            .args(flags)
            .arg(format!("--offload-arch={arch}"))
            .arg("-I")
            .arg(&include_dir)
            .args(["-x", "hip", "-c"])
            .arg(&path)
            .arg("-o")
            .arg(&obj));
        println!("cargo:rerun-if-changed={}", path.display());
        objects.push(obj);
    }
    for header in [
        "csrc/device.h",
        "csrc/gemm.h",
        "csrc/kernels.h",
        "csrc/internal.h",
        "csrc/q35.h",
        "csrc/expf.h",
        "csrc/log1pf.h",
    ] {
        println!("cargo:rerun-if-changed={}", src_dir.join(header).display());
    }
    println!("cargo:rerun-if-changed={}", src_dir.join("build.manifest").display());
    println!("cargo:rerun-if-changed={}", include_dir.join("cohx.h").display());

    // -z defs: a symbol the host pass dropped fails here, not at load time
    let lib = out.join("libcohx.so");
    run(Command::new(&hipcc)
        .arg(format!("--offload-arch={arch}"))
        .args(["-shared", "-fPIC", "-Wl,-z,defs", "-o"])
        .arg(&lib)
        .args(&objects)
        .args(section(&m, "link")));

    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=cohx");
    // the library is found next to the binary's build output at run time
    println!("cargo:rustc-link-arg=-Wl,-rpath,{}", out.display());
    for var in ["COHX_SRC_DIR", "COHX_INCLUDE_DIR", "HIPCC", "COHX_ARCH"] {
        println!("cargo:rerun-if-env-changed={var}");
    }
}

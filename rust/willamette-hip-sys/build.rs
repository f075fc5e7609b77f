//! Builds libwillamette_hip.so with hipcc for gfx950 (the same sources and
//! flags as project-willamette_amd/build.py), or links a prebuilt one from
//! WILLAMETTE_HIP_LIB_DIR.

use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;

const FLAGS: &[&str] = &[
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "--offload-arch=gfx950",
];

/// Extra flags of single sources (as PER_FILE in build.py): the batched GEMM
/// keeps its MFMA accumulators in VGPRs; the fused matvecs and decode
/// attention take what their first loads need in their leading 16 argument
/// dwords, preloaded into SGPRs at wave launch.
fn per_file(name: &str) -> &'static [&'static str] {
    match name {
        "k_batch.hip" => &["-mllvm", "-amdgpu-mfma-vgpr-form"],
        "k_i2s.hip" | "k_attn.hip" => &["-mllvm", "-amdgpu-kernarg-preload-count=16"],
        _ => &[],
    }
}

fn main() {
    println!("cargo:rerun-if-env-changed=WILLAMETTE_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=HIPCC");
    if let Ok(dir) = env::var("WILLAMETTE_HIP_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-lib=dylib=willamette_hip");
        return;
    }
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let repo = manifest.join("../..").canonicalize().expect("repository root");
    let csrc = repo.join("project-willamette_amd/csrc");
    let include = repo.join("include");
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".to_string());

    let mut sources: Vec<PathBuf> = std::fs::read_dir(&csrc)
        .expect("csrc directory")
        .filter_map(|e| e.ok().map(|e| e.path()))
        .filter(|p| matches!(p.extension().and_then(|e| e.to_str()), Some("hip") | Some("cpp")))
        .collect();
    sources.sort();
    println!("cargo:rerun-if-changed={}", csrc.display());
    println!("cargo:rerun-if-changed={}", include.display());

    let mut objects = Vec::new();
    for src in &sources {
        let obj = out.join(format!("{}.o", src.file_name().unwrap().to_string_lossy()));
        let mut cmd = Command::new(&hipcc);
        cmd.args(FLAGS).args(per_file(&src.file_name().unwrap().to_string_lossy()));
        cmd.arg("-I").arg(&include).arg("-I").arg(&csrc);
        if src.extension().and_then(|e| e.to_str()) == Some("hip") {
            cmd.arg("-x").arg("hip");
        }
        cmd.arg("-c");
        cmd.arg(src).arg("-o").arg(&obj);
        run(&mut cmd, src);
        objects.push(obj);
    }
    let lib = out.join("libwillamette_hip.so");
    let mut link = Command::new(&hipcc);
    link.arg("--offload-arch=gfx950").arg("-shared").args(&objects).arg("-o").arg(&lib).arg("-lpthread");
    run(&mut link, &lib);
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=willamette_hip");
}

fn run(cmd: &mut Command, what: &Path) {
    let status = cmd.status().unwrap_or_else(|e| panic!("hipcc for {}: {e}", what.display()));
    assert!(status.success(), "hipcc failed for {}", what.display());
}

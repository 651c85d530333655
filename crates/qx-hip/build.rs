//! Compiles the HIP sources of qx_amd/csrc for gfx950 into libqx_hip.so, as
//! qx_amd/build.py does, and links it.  QX_HIP_SRC points at qx_amd/csrc
//! (default: ../../qx_amd/csrc relative to this crate); ROCM_PATH at the ROCm
//! install (default /opt/rocm).
use std::{env, path::PathBuf, process::Command};

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let src = env::var("QX_HIP_SRC")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("../../qx_amd/csrc"));
    let rocm = PathBuf::from(env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into()));
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let hipcc = rocm.join("bin/hipcc");
    let mut objects = Vec::new();
    let mut sources: Vec<PathBuf> = std::fs::read_dir(&src)
        .unwrap_or_else(|e| panic!("QX_HIP_SRC {}: {e}", src.display()))
        .map(|entry| entry.unwrap().path())
        .collect();
    sources.sort();
    for path in sources {
        println!("cargo:rerun-if-changed={}", path.display());
        if path.extension().map_or(true, |e| e != "hip") {
            continue;
        }
        let obj = out.join(path.file_name().unwrap()).with_extension("o");
        let status = Command::new(&hipcc)
            .args([
                "--offload-arch=gfx950",
                "-O3",
                "-std=c++17",
                "-fPIC",
                "-ffp-contract=off",
                "-fvisibility=hidden",
                "-Xclang",
                "-target-feature",
                "-Xclang",
                "-packed-fp32-ops",
                "-c",
            ])
            .arg(&path)
            .arg("-o")
            .arg(&obj)
            .status()
            .expect("hipcc");
        assert!(status.success(), "hipcc failed on {}", path.display());
        objects.push(obj);
    }
    let lib = out.join("libqx_hip.so");
    let status = Command::new(&hipcc)
        .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
        .arg(&lib)
        .args(&objects)
        .status()
        .expect("hipcc link");
    assert!(status.success(), "link of libqx_hip.so failed");
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=qx_hip");
    println!("cargo:rustc-link-search=native={}", rocm.join("lib").display());
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rerun-if-env-changed=QX_HIP_SRC");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}

// The `hip` feature of det-sys: compiles kernels/hip (this repository's det_amd/csrc/*.hip and include/det_hip.h)
// with hipcc for gfx950 into a static library and links the HIP runtime.  build.rs calls build_hip(&kernels.join("hip"))
// when CARGO_FEATURE_HIP is set (exclusive with metal and cuda), next to its build_cuda (reference
// crates/det-sys/build.rs:93-145).  UNVERIFIED: no Rust toolchain was available where this was written.
//
// Flags: the spec's numerics need every fp32 operation as written -- no contraction, no fast math, denormals kept,
// correctly rounded division and square root; packed fp32 VALU ops are kept out of the generated code.
use std::path::{Path, PathBuf};
use std::process::Command;

fn build_hip(kernels: &Path) {
    let rocm = std::env::var_os("ROCM_PATH").map(PathBuf::from).unwrap_or_else(|| PathBuf::from("/opt/rocm"));
    let arch = std::env::var("DET_HIP_ARCH").unwrap_or_else(|_| "gfx950".into());
    let out = PathBuf::from(std::env::var("OUT_DIR").unwrap());
    let hipcc = rocm.join("bin/hipcc");
    let mut sources: Vec<PathBuf> = std::fs::read_dir(kernels)
        .unwrap()
        .map(|e| e.unwrap().path())
        .filter(|p| p.extension().is_some_and(|x| x == "hip"))
        .collect();
    sources.sort();
    let mut objects = Vec::new();
    for src in &sources {
        let obj = out.join(src.file_stem().unwrap()).with_extension("o");
        let status = Command::new(&hipcc)
            .args([&format!("--offload-arch={arch}"), "-O3", "-std=c++17", "-fPIC", "-c"])
            .args(["-ffp-contract=off", "-fno-fast-math", "-fno-gpu-flush-denormals-to-zero"])
            .arg("-fhip-fp32-correctly-rounded-divide-sqrt")
            .args(["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"])
            .args(["-mllvm", "-amdgpu-mfma-vgpr-form=1"])
            .arg("-I")
            .arg(kernels)
            .arg(src)
            .arg("-o")
            .arg(&obj)
            .status()
            .expect("hipcc not found: set ROCM_PATH");
        assert!(status.success(), "hipcc failed on {}", src.display());
        objects.push(obj);
    }
    let lib = out.join("libdet_hip.a");
    let _ = std::fs::remove_file(&lib);
    let status = Command::new("ar").arg("crs").arg(&lib).args(&objects).status().unwrap();
    assert!(status.success(), "ar failed");
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=static=det_hip");
    println!("cargo:rustc-link-search=native={}", rocm.join("lib").display());
    for l in ["amdhip64", "stdc++", "dl", "pthread"] {
        println!("cargo:rustc-link-lib={l}");
    }
    for s in &sources {
        println!("cargo:rerun-if-changed={}", s.display());
    }
    for h in ["det_hip.h", "common.h", "gemm_common.h", "gemm_internal.h", "mixer_internal.h", "gguf_reader.h"] {
        println!("cargo:rerun-if-changed={}", kernels.join(h).display());
    }
    for v in ["ROCM_PATH", "DET_HIP_ARCH"] {
        println!("cargo:rerun-if-env-changed={v}");
    }
}

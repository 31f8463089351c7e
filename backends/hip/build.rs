//! Compiles libqi_hip.so for gfx950 with hipcc and links it.
//!
//! The translation units are read from `sources.txt` in the source directory
//! (`QI_HIP_SRC`, default `../../quantinfer_amd/csrc` from this crate), the
//! list quantinfer_amd/build.py builds from, so the two builds compile the
//! same files. The flags are build.py's: gfx950 only, no FMA contraction, no
//! fast-math, f32 denormals kept, packed FP32 instructions off, and the same
//! per-file additions (the GEMV keeps its matrix-instruction results in
//! ordinary VGPRs).
use std::{env, fs, path::PathBuf, process::Command};

const FLAGS: &[&str] = &[
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
];

const FILE_FLAGS: &[(&str, &[&str])] = &[
    ("qi_gemv_mfma.hip", &["-mllvm", "-amdgpu-mfma-vgpr-form"]),
    ("qi_gemv_rows.hip", &["-mllvm", "-amdgpu-mfma-vgpr-form"]),
    ("qi_gemv_rm.hip", &["-mllvm", "-amdgpu-mfma-vgpr-form"]),
];

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").unwrap());
    let src = env::var("QI_HIP_SRC")
        .map(PathBuf::from)
        .unwrap_or_else(|_| manifest.join("../../quantinfer_amd/csrc"));
    let list = fs::read_to_string(src.join("sources.txt")).expect("sources.txt lists the HIP sources");
    let sources: Vec<&str> = list
        .lines()
        .map(str::trim)
        .filter(|l| !l.is_empty() && !l.starts_with('#'))
        .collect();
    let out = PathBuf::from(env::var("OUT_DIR").unwrap());
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".into());
    let mut objects = Vec::new();
    for file in &sources {
        let obj = out.join(format!("{file}.o"));
        let mut cmd = Command::new(&hipcc);
        if file.ends_with(".cpp") {
            // host code in the same HIP translation model
            cmd.args(["-x", "hip"]);
        }
        cmd.args(FLAGS);
        for (name, extra) in FILE_FLAGS {
            if name == file {
                cmd.args(*extra);
            }
        }
        let status = cmd
            .arg("-c")
            .arg(src.join(file))
            .arg("-o")
            .arg(&obj)
            .status()
            .expect("hipcc is required to build the HIP backend");
        assert!(status.success(), "hipcc failed on {file}");
        objects.push(obj);
        println!("cargo:rerun-if-changed={}", src.join(file).display());
    }
    let lib = out.join("libqi_hip.so");
    let status = Command::new(&hipcc)
        .args(["--offload-arch=gfx950", "-shared", "-fPIC", "-o"])
        .arg(&lib)
        .args(&objects)
        .args(["-Wl,-rpath,/opt/rocm/lib"])
        .status()
        .expect("hipcc link");
    assert!(status.success(), "linking libqi_hip.so failed");
    println!("cargo:rerun-if-changed={}", src.join("sources.txt").display());
    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=qi_hip");
}

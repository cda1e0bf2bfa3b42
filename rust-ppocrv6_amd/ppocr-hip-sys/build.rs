//! Builds libppocr_rechead.so from ../csrc with hipcc, for gfx950 (MI355X) only, into
//! OUT_DIR, and links it.  One hipcc process per source file, run in parallel; the same
//! flags as csrc/Makefile (packed fp32 instructions off for device code).
//!
//! Environment: HIPCC (default /opt/rocm/bin/hipcc).  Dependents' build scripts find the
//! library's directory in DEP_PPOCR_RECHEAD_ROOT (the `links` key), e.g. to set an rpath.
use std::env;
use std::path::{Path, PathBuf};
use std::process::Command;
use std::thread;

const SOURCES: &[&str] = &[
    "api.hip",
    "pack.hip",
    "prep.hip",
    "head_mfma.hip",
    "head_cfg_q.hip",
    "head_cfg_f.hip",
    "head_cfg_h.hip",
    "head_cfg_rescue.hip",
    "head_fma.hip",
    "softmax_ctc.hip",
    "neck.hip",
    "safetensors.cpp",
    "model_graph.cpp",
];
const HEADERS: &[&str] =
    &["common.hpp", "kernels.hpp", "neck.hpp", "head_mfma.hpp", "safetensors.hpp", "json.hpp", "model_graph.hpp"];
const FLAGS: &[&str] = &[
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
];

// Per-file flags: the tail's kernels keep MFMA results in ordinary vector registers (no
// accumulator-register copies before their vector work).
fn file_flags(src: &str) -> &'static [&'static str] {
    if src == "neck.hip" {
        &["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
    } else {
        &[]
    }
}

fn run(cmd: &mut Command) {
    let status = cmd.status().unwrap_or_else(|e| panic!("failed to start {:?}: {}", cmd, e));
    if !status.success() {
        panic!("{:?} failed with {}", cmd, status);
    }
}

fn main() {
    let manifest = PathBuf::from(env::var("CARGO_MANIFEST_DIR").expect("CARGO_MANIFEST_DIR"));
    let csrc = manifest.join("..").join("csrc");
    let header = manifest.join("..").join("..").join("include").join("ppocr_rechead.h");
    let out = PathBuf::from(env::var("OUT_DIR").expect("OUT_DIR"));
    let hipcc = env::var("HIPCC").unwrap_or_else(|_| "/opt/rocm/bin/hipcc".to_string());

    let jobs: Vec<_> = SOURCES
        .iter()
        .map(|src| {
            let (hipcc, csrc, out) = (hipcc.clone(), csrc.clone(), out.clone());
            let src = src.to_string();
            thread::spawn(move || {
                let obj = out.join(format!("{}.o", src));
                run(Command::new(&hipcc)
                    .args(FLAGS)
                    .args(file_flags(&src))
                    .arg("-c")
                    .arg(csrc.join(&src))
                    .arg("-o")
                    .arg(&obj));
                obj
            })
        })
        .collect();
    let objs: Vec<PathBuf> = jobs.into_iter().map(|j| j.join().expect("compile thread")).collect();

    let lib = out.join("libppocr_rechead.so");
    run(Command::new(&hipcc).args(FLAGS).arg("-shared").args(&objs).arg("-o").arg(&lib));

    println!("cargo:rustc-link-search=native={}", out.display());
    println!("cargo:rustc-link-lib=dylib=ppocr_rechead");
    println!("cargo:root={}", out.display());
    println!("cargo:rerun-if-env-changed=HIPCC");
    for f in SOURCES.iter().chain(HEADERS.iter()) {
        println!("cargo:rerun-if-changed={}", csrc.join(f).display());
    }
    println!("cargo:rerun-if-changed={}", Path::new(&header).display());
}

// Links the prebuilt libfracture_hip.so (and the HIP runtime and rocBLAS it depends on).
// FRACTURE_HIP_LIB_DIR names the directory holding the library (fracture_amd/ after
// `python -m fracture_amd.build`); ROCM_PATH defaults to /opt/rocm.
fn main() {
    let dir = std::env::var("FRACTURE_HIP_LIB_DIR")
        .expect("set FRACTURE_HIP_LIB_DIR to the directory of libfracture_hip.so");
    let rocm = std::env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".into());
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=fracture_hip");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rustc-link-lib=dylib=rocblas");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    println!("cargo:rerun-if-env-changed=FRACTURE_HIP_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}

// Links librtensor_hip.so, built by `python -m rgpu_amd.build` (hipcc
// --offload-arch=gfx950).  RTENSOR_HIP_DIR names the directory that holds it.
fn main() {
    println!("cargo:rerun-if-env-changed=RTENSOR_HIP_DIR");
    let dir = std::env::var("RTENSOR_HIP_DIR")
        .expect("set RTENSOR_HIP_DIR to the directory of librtensor_hip.so");
    println!("cargo:rustc-link-search=native={dir}");
    println!("cargo:rustc-link-lib=dylib=rtensor_hip");
}

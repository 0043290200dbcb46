// Links libema_attn.so (built by `make -C engine-mlx_amd`, into engine-mlx_amd/ema_attn/)
// and the HIP runtime it runs on.
//   EMA_ATTN_LIB_DIR  directory holding libema_attn.so (default /opt/ema_attn/lib)
//   ROCM_PATH         ROCm install (default /opt/rocm), for libamdhip64.so
use std::env;

fn main() {
    let lib_dir = env::var("EMA_ATTN_LIB_DIR").unwrap_or_else(|_| "/opt/ema_attn/lib".to_string());
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_string());
    println!("cargo:rustc-link-search=native={lib_dir}");
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=ema_attn");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{lib_dir}");
    println!("cargo:rerun-if-env-changed=EMA_ATTN_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
}

// Links librunit_hip.so, the host runtime of the MI355X kernels
// (built by `python -c "import __graft_entry__ as g; g.build()"` at the
// repository root, into runit_mac_amd/lib/).
fn main() {
    let lib = std::env::var("RUNIT_HIP_LIB").unwrap_or_else(|_| {
        let here = std::env::var("CARGO_MANIFEST_DIR").unwrap();
        format!("{here}/../../runit_mac_amd/lib")
    });
    println!("cargo:rerun-if-env-changed=RUNIT_HIP_LIB");
    println!("cargo:rustc-link-search=native={lib}");
    println!("cargo:rustc-link-lib=dylib=runit_hip");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{lib}");
}

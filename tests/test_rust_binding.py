"""CPU checks of the Rust binding (burn-rocket_amd/rust/), which this image cannot
compile: the `extern "C"` block of rocket-hip-sys declares exactly the entry
points of include/burn_rocket_amd.h, with the same arity, pointer kinds and
constness per parameter and the same return type; its constants equal the
header's; and every `hip::` item the replacement `impl RocketOps for Flex`
uses exists in the crate."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "burn_rocket_amd.h")
SYS = os.path.join(ROOT, "burn-rocket_amd", "rust", "rocket-hip-sys", "src", "lib.rs")
EXT = os.path.join(ROOT, "burn-rocket_amd", "rust", "burn-rocket-ext", "ext_hip.rs")


def _header_fns():
    t = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    t = re.sub(r"#.*", "", t)
    out = {}
    for m in re.finditer(r"\b(int|const char \*)\s*(rk_\w+)\s*\(([^)]*)\)\s*;", t):
        params = [] if m.group(3).strip() == "void" else [" ".join(p.split()) for p in m.group(3).split(",")]
        kinds = []
        for p in params:
            name = re.findall(r"(\w+)$", p)[0]
            ty = p[:p.rfind(name)]
            kinds.append((ty.count("*"), ty.strip().startswith("const")))
        out[m.group(2)] = ("int" if m.group(1) == "int" else "str", kinds)
    return out


def _rust_fns():
    t = open(SYS).read()
    block = t[t.index('unsafe extern "C" {'):]
    block = block[:block.index("\n}\n")]
    out = {}
    for m in re.finditer(r"pub fn (rk_\w+)\((.*?)\)\s*->\s*([^;]+);", block, flags=re.S):
        params = [p.strip() for p in " ".join(m.group(2).split()).split(",") if p.strip()]
        kinds = []
        for p in params:
            ty = p.split(":", 1)[1].strip()
            stars = ty.count("*")
            kinds.append((stars, ty.startswith("*const")))
        out[m.group(1)] = ("int" if m.group(3).strip() == "c_int" else "str", kinds)
    return out


def test_extern_block_matches_the_header():
    h, r = _header_fns(), _rust_fns()
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name in h:
        assert h[name][0] == r[name][0], f"{name}: return type"
        assert len(h[name][1]) == len(r[name][1]), f"{name}: arity {len(h[name][1])} vs {len(r[name][1])}"
        for i, (hk, rk) in enumerate(zip(h[name][1], r[name][1])):
            # rk_stream is a pointer type in Rust (Stream = *mut c_void) and a typedef in C
            if hk[0] == 0 and rk[0] == 1 and not rk[1]:
                continue
            assert hk == rk, f"{name} parameter {i}: C {hk} vs Rust {rk}"


def test_constants_match_the_header():
    defines = dict(re.findall(r"#define (RK_\w+) \(?(-?\w+)", open(HEADER).read()))
    rust = dict(re.findall(r"pub const (RK_\w+): \w+ = (-?\w+)", open(SYS).read()))
    for name, val in rust.items():
        if name == "RK_NOALLOC_SCRATCH_BYTES":
            assert "(32u << 20)" in open(HEADER).read() and val == "32"
            continue
        assert defines[name] == val, name
    for name in ("RK_OK", "RK_E_SHAPE", "RK_E_TILING", "RK_E_NOMEM", "RK_E_DEVICE", "RK_E_UNSUPPORTED",
                 "RK_E_RANGE", "RK_E_IO", "RK_MASK_NONE", "RK_MASK_CAUSAL", "RK_MASK_WINDOW",
                 "RK_MASK_CAUSAL_WINDOW"):
        assert name in rust, name


def test_wrappers_and_the_flex_impl_use_declared_items():
    sys_src = open(SYS).read()
    declared = set(_rust_fns())
    wrappers = sys_src[sys_src.index("/// A failed call"):]
    for name in set(re.findall(r"\b(rk_\w+)\(", wrappers)):
        assert name in declared, name
    items = set(re.findall(r"pub (?:fn|const|struct|type) (\w+)", sys_src))
    used = set(re.findall(r"\bhip::(\w+)", open(EXT).read()))
    assert used and used <= items, sorted(used - items)
    # every op of the reference trait (ext.rs:57-164) is implemented
    ext = open(EXT).read()
    for op in ("rocket_pack", "rocket_pack2", "rocket_pack3", "rocket_pack_i8", "rocket_gelu_mul",
               "rocket_silu_mul", "rocket_rms_norm", "rocket_rms_norm_noscale", "rocket_rope", "rocket_matmul",
               "rocket_attention", "rocket_attention_window", "rocket_attention_causal_window",
               "rocket_attention_window_block", "rocket_attention_causal_block"):
        assert re.search(rf"fn {op}\(", ext), op

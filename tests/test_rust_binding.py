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


CTX = os.path.join(ROOT, "burn-rocket_amd", "rust", "rocket-hip-sys", "src", "ctx.rs")
NPU = os.path.join(ROOT, "burn-rocket_amd", "rust", "rocket-hip-sys", "src", "npu.rs")


def _split_params(params):
    out, depth, cur = [], 0, ""
    for ch in params:
        if ch in "<([":
            depth += 1
        elif ch in ">)]":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return [p for p in out if p not in ("&self", "&mut self", "self", "mut self")]


def _methods(path, type_name=None):
    """name -> number of parameters (self excluded) of the `pub fn`s of `impl
    type_name` (or of the file's free functions when type_name is None)."""
    src = re.sub(r"//.*", "", open(path).read())
    if type_name is not None:
        start = src.index(f"impl {type_name} {{")
        depth, i = 0, src.index("{", start)
        for j in range(i, len(src)):
            depth += {"{": 1, "}": -1}.get(src[j], 0)
            if depth == 0:
                break
        src = src[i:j]
    out = {}
    for m in re.finditer(r"pub (?:const )?fn (\w+)\s*\((.*?)\)\s*(->|\{)", src, flags=re.S):
        out[m.group(1)] = len(_split_params(" ".join(m.group(2).split())))
    return out


# The signatures a drop-in must keep (the Rust API the app calls), with the
# reference's parameter counts, self excluded.
KEEP = [
    # free functions of crates/burn-rocket/src/ext.rs whose bodies reach the engine
    (EXT, None, {"init": 1,            # ext.rs:561
                 "pack_qat": 6,        # ext.rs:1382-1389
                 "stats": 0, "stats_reset": 0,            # ext.rs:186-200
                 "mem_stats": 0,       # ext.rs:206
                 "trim_scratch": 0,    # ext.rs:254
                 "trim_scratch_to": 1,  # ext.rs:281
                 "clear_scratch": 0}),  # ext.rs:266
    # RocketCtx / RocketFaCtx, crates/burn-rocket/src/lib.rs:203-330
    (CTX, "RocketCtx", {"new": 1, "pack_weight": 4, "pack_weight_seg": 3, "matmul_prepacked": 6,
                        "trim_scratch": 0, "trim_to_budget": 1, "scratch_bytes": 0, "clear_scratch": 0,
                        "mem_stats": 0}),
    (CTX, "RocketFaCtx", {"new": 1, "flash_attn": 13, "mem_stats": 0}),
    (CTX, "RocketWeight", {"bytes": 0}),
    # I8Context / I8Weight, crates/rocket-npu/src/matmul/int8.rs:126-676
    (NPU, "I8Context", {"new": 1, "new_at": 2, "pack_weight": 4, "pack_weight_gw": 5, "rewrite_weight": 2,
                        "rewrite_weight_gw": 2, "matmul": 6, "matmul_gw": 8, "scratch_bytes": 0,
                        "clear_scratch": 0}),
    (NPU, "I8Weight", {"shape": 0, "bytes": 0}),
    # rocket_npu::Error accessors used by Clef (src/clef/engine_npu.rs:63-71), error.rs:69-150
    (NPU, "Error", {"op": 0, "status": 0, "errno": 0, "c_code": 0}),
    (NPU, "Status", {"code": 0, "from_code": 1}),
]


def test_the_reference_signatures_are_kept():
    for path, ty, want in KEEP:
        got = _methods(path, ty)
        for name, arity in want.items():
            assert name in got, f"{os.path.basename(path)} {ty or ''}::{name} missing"
            assert got[name] == arity, f"{ty or ''}::{name}: {got[name]} parameters, the reference has {arity}"


def test_safe_wrappers_check_output_lengths():
    # Every safe wrapper that hands a mutable slice to the library checks its
    # length first (a short slice would be written past its end).
    src = open(SYS).read()
    body = src[src.index("/// A failed call"):]
    for m in re.finditer(r"pub fn (\w+)\s*(?:<[^>]*>)?\((.*?)\)\s*->[^{]*\{(.*?)\n\}", body, flags=re.S):
        name, params, fn_body = m.groups()
        outs = re.findall(r"(\w+): &mut \[", params)
        for o in outs:
            assert re.search(rf"\b{o}\.len\(\)", fn_body), f"{name}: no length check on {o}"

"""The Java 21 FFM binding (gpullama3.java_amd/java) against the C ABI, on the CPU.

No JDK exists in this environment, so the Java sources are checked as text:
every downcall descriptor in Gl3.java must be the C signature of the function
of the same name in include/gl3.h (pointer -> ADDRESS, int / int32_t /
uint32_t -> JAVA_INT, size_t / int64_t / uint64_t -> JAVA_LONG, float ->
JAVA_FLOAT), every constant must equal the header's, only Java 21 FFM names may
be used (getUtf8String / allocateUtf8String / allocateArray; not the Java 22
getString / allocateFrom / allocate(layout, count)), and the master plan must
keep the reference's public signatures (TornadoVMMasterPlan.java:37,127,180,200)
with no TornadoVM import left.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JAVA = os.path.join(ROOT, "gpullama3.java_amd", "java", "src", "main", "java", "org", "beehive", "gpullama3")
HEADER = os.path.join(ROOT, "include", "gl3.h")

C_TO_LAYOUT = {"int": "JAVA_INT", "int32_t": "JAVA_INT", "uint32_t": "JAVA_INT", "size_t": "JAVA_LONG",
               "int64_t": "JAVA_LONG", "uint64_t": "JAVA_LONG", "float": "JAVA_FLOAT", "double": "JAVA_DOUBLE"}


def java_sources():
    out = {}
    for d, _, files in os.walk(JAVA):
        for f in files:
            if f.endswith(".java"):
                p = os.path.join(d, f)
                out[os.path.relpath(p, JAVA)] = open(p).read()
    return out


def strip_c_comments(src):
    return re.sub(r"/\*.*?\*/", "", src, flags=re.S)


def c_layout(decl):
    decl = decl.strip()
    if "*" in decl:
        return "ADDRESS"
    words = [w for w in re.findall(r"[A-Za-z_][A-Za-z0-9_]*", decl) if w not in ("const", "unsigned", "struct")]
    return C_TO_LAYOUT[words[0]]


def header_functions():
    src = strip_c_comments(open(HEADER).read())
    src = re.sub(r"#.*", "", src)
    funcs = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(gl3_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", src, flags=re.S):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        ret = ret.split(";")[-1].split("}")[-1].strip()
        args = [] if params.strip() in ("", "void") else [c_layout(re.sub(r"\b\w+\s*$", "", a.strip()) if not
                                                                   a.strip().endswith("*") else a) for a in
                                                          params.split(",")]
        funcs[name] = ("VOID" if ret == "void" else c_layout(ret), args)
    return funcs


def java_descriptors():
    src = java_sources()[os.path.join("hip", "Gl3.java")]
    out = {}
    for m in re.finditer(r'fn\("(gl3_[a-z0-9_]+)",\s*FunctionDescriptor\.(of|ofVoid)\(([^;]*?)\)\);', src, flags=re.S):
        name, kind, body = m.group(1), m.group(2), m.group(3)
        toks = [t.strip() for t in body.split(",") if t.strip()]
        out[name] = ("VOID", toks) if kind == "ofVoid" else (toks[0], toks[1:])
    return out


def test_every_header_function_has_a_matching_downcall():
    h, j = header_functions(), java_descriptors()
    assert {"gl3_create", "gl3_forward", "gl3_prefill", "gl3_generate_sampled", "gl3_op_attention_noalloc"} <= set(h)
    assert sorted(h) == sorted(j), (sorted(set(h) ^ set(j)))
    for name in h:
        assert h[name] == j[name], (name, h[name], j[name])


def header_int(name):
    src = open(HEADER).read()
    m = re.search(rf"\b{name}\s*=\s*(\d+)", src) or re.search(rf"#define\s+{name}\s+(\d+)u?\b", src)
    assert m, name
    return int(m.group(1))


@pytest.mark.parametrize("java_name,c_name", [
    ("ABI_VERSION", "GL3_ABI_VERSION"), ("OK", "GL3_OK"), ("ERR_INVALID_ARGUMENT", "GL3_ERR_INVALID_ARGUMENT"),
    ("ERR_UNSUPPORTED", "GL3_ERR_UNSUPPORTED"), ("ERR_OUT_OF_MEMORY", "GL3_ERR_OUT_OF_MEMORY"),
    ("ERR_DEVICE", "GL3_ERR_DEVICE"), ("ERR_STATE", "GL3_ERR_STATE"),
    ("MODEL_LLAMA_3", "GL3_MODEL_LLAMA_3"), ("MODEL_MISTRAL", "GL3_MODEL_MISTRAL"),
    ("MODEL_QWEN_3", "GL3_MODEL_QWEN_3"), ("MODEL_PHI_3", "GL3_MODEL_PHI_3"), ("MODEL_QWEN_2", "GL3_MODEL_QWEN_2"),
    ("MODEL_DEEPSEEK_R1_DISTILL_QWEN", "GL3_MODEL_DEEPSEEK_R1_DISTILL_QWEN"),
    ("TYPE_F32", "GL3_TYPE_F32"), ("TYPE_F16", "GL3_TYPE_F16"), ("TYPE_Q8_0", "GL3_TYPE_Q8_0"),
    ("TOKEN_EMBD", "GL3_TOKEN_EMBD"), ("OUTPUT_NORM", "GL3_OUTPUT_NORM"), ("OUTPUT", "GL3_OUTPUT"),
    ("ATTN_NORM", "GL3_ATTN_NORM"), ("ATTN_Q", "GL3_ATTN_Q"), ("ATTN_K", "GL3_ATTN_K"), ("ATTN_V", "GL3_ATTN_V"),
    ("ATTN_QKV", "GL3_ATTN_QKV"), ("ATTN_OUTPUT", "GL3_ATTN_OUTPUT"), ("ATTN_Q_NORM", "GL3_ATTN_Q_NORM"),
    ("ATTN_K_NORM", "GL3_ATTN_K_NORM"), ("FFN_NORM", "GL3_FFN_NORM"), ("FFN_GATE", "GL3_FFN_GATE"),
    ("FFN_UP", "GL3_FFN_UP"), ("FFN_DOWN", "GL3_FFN_DOWN"),
    ("FLAG_PHASE_KERNELS", "GL3_FLAG_PHASE_KERNELS"), ("FLAG_TIMING", "GL3_FLAG_TIMING"),
    ("FLAG_PHASE_TRACE", "GL3_FLAG_PHASE_TRACE"), ("FLAG_STEPWISE_PROMPT", "GL3_FLAG_STEPWISE_PROMPT"),
    ("GEMV_STORE", "GL3_GEMV_STORE"), ("GEMV_RESIDUAL", "GL3_GEMV_RESIDUAL"), ("GEMV_SWIGLU", "GL3_GEMV_SWIGLU"),
])
def test_constants_match_the_header(java_name, c_name):
    src = java_sources()[os.path.join("hip", "Gl3.java")]
    m = re.search(rf"static final int {java_name}\s*=\s*(\d+);", src)
    assert m, java_name
    assert int(m.group(1)) == header_int(c_name)


def test_config_layout_matches_the_header():
    src = java_sources()[os.path.join("hip", "Gl3.java")]
    body = re.search(r"CONFIG = MemoryLayout\.structLayout\((.*?)\);", src, re.S).group(1)
    java_fields = re.findall(r'(JAVA_\w+)\.withName\("(\w+)"\)', body)
    hbody = re.search(r"typedef struct gl3_config \{(.*?)\} gl3_config;", open(HEADER).read(), re.S).group(1)
    hbody = strip_c_comments(hbody)
    c_fields = [(C_TO_LAYOUT[t], n) for t, n in re.findall(r"\b(int32_t|uint32_t|float)\s+(\w+);", hbody)]
    assert java_fields == c_fields
    assert "NOALLOC_SCRATCH_BYTES = 1280L << 10" in src
    assert "(1280u << 10)" in open(HEADER).read()


def test_only_java21_ffm_names():
    for rel, src in java_sources().items():
        code = re.sub(r"//.*|/\*.*?\*/", "", src, flags=re.S)
        assert ".getString(" not in code, rel
        assert "allocateFrom(" not in code, rel
        assert not re.search(r"\.allocate\(\s*JAVA_\w+\s*,", code), rel  # Java 22 allocate(layout, count)
        assert "uk.ac.manchester.tornado" not in code, rel


def test_master_plan_keeps_the_reference_signatures():
    src = java_sources()[os.path.join("tornadovm", "TornadoVMMasterPlan.java")]
    for sig in (r"public static TornadoVMMasterPlan initializeTornadoVMPlan\(State state, Model model\)",
                r"public FloatTensor tornadoVMForwardExecuteLayered\(int position\)",
                r"public void forceCopyInReadOnlyDataLayered\(\)",
                r"public void freeTornadoExecutionPlan\(\)",
                r"public TornadoVMMasterPlan\(State state, Model model\)",
                r"public static final boolean ENABLE_TORNADOVM_INIT_TIME"):
        assert re.search(sig, src), sig


def test_every_handle_used_is_declared():
    srcs = java_sources()
    declared = set(java_descriptors())
    for rel, src in srcs.items():
        for name in re.findall(r"Gl3\.(gl3_[a-z0-9_]+)", src):
            assert name in declared, (rel, name)

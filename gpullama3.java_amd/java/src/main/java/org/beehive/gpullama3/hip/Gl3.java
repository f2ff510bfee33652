package org.beehive.gpullama3.hip;

import java.lang.foreign.Arena;
import java.lang.foreign.FunctionDescriptor;
import java.lang.foreign.Linker;
import java.lang.foreign.MemoryLayout;
import java.lang.foreign.MemorySegment;
import java.lang.foreign.StructLayout;
import java.lang.foreign.SymbolLookup;
import java.lang.invoke.MethodHandle;

import static java.lang.foreign.MemoryLayout.PathElement.groupElement;
import static java.lang.foreign.ValueLayout.ADDRESS;
import static java.lang.foreign.ValueLayout.JAVA_FLOAT;
import static java.lang.foreign.ValueLayout.JAVA_INT;
import static java.lang.foreign.ValueLayout.JAVA_LONG;

/**
 * Downcalls into libgpullama3_hip.so, one method handle per function of
 * include/gl3.h, written against the Foreign Function & Memory API of Java 21
 * (JEP 442, a preview there: the reference builds with --enable-preview,
 * pom.xml:75).  The library path comes from -Dgl3.library (default: the
 * loader's search for libgpullama3_hip.so).
 *
 * <p>Every entry point returns a status; {@link #check(int)} turns a failure
 * into the exception the reference would raise for the same condition, with
 * the library's thread-local message.
 */
public final class Gl3 {
    private Gl3() {
    }

    public static final int ABI_VERSION = 1;

    // gl3_status
    public static final int OK = 0;
    public static final int ERR_INVALID_ARGUMENT = 1;
    public static final int ERR_UNSUPPORTED = 2;
    public static final int ERR_OUT_OF_MEMORY = 3;
    public static final int ERR_DEVICE = 4;
    public static final int ERR_STATE = 5;

    // gl3_model_type: the order of the reference's ModelType (model/ModelType.java:24-80)
    public static final int MODEL_LLAMA_3 = 0;
    public static final int MODEL_MISTRAL = 1;
    public static final int MODEL_QWEN_3 = 2;
    public static final int MODEL_PHI_3 = 3;
    public static final int MODEL_QWEN_2 = 4;
    public static final int MODEL_DEEPSEEK_R1_DISTILL_QWEN = 5;

    // gl3_ggml_type: GGMLType ordinals (tensor/GGMLType.java)
    public static final int TYPE_F32 = 0;
    public static final int TYPE_F16 = 1;
    public static final int TYPE_Q8_0 = 8;

    // gl3_tensor_kind
    public static final int TOKEN_EMBD = 0;
    public static final int OUTPUT_NORM = 1;
    public static final int OUTPUT = 2;
    public static final int ATTN_NORM = 3;
    public static final int ATTN_Q = 4;
    public static final int ATTN_K = 5;
    public static final int ATTN_V = 6;
    public static final int ATTN_QKV = 7;
    public static final int ATTN_OUTPUT = 8;
    public static final int ATTN_Q_NORM = 9;
    public static final int ATTN_K_NORM = 10;
    public static final int FFN_NORM = 11;
    public static final int FFN_GATE = 12;
    public static final int FFN_UP = 13;
    public static final int FFN_DOWN = 14;

    // plan flags
    public static final int FLAG_PHASE_KERNELS = 1;
    public static final int FLAG_TIMING = 2;
    public static final int FLAG_PHASE_TRACE = 4;
    public static final int FLAG_STEPWISE_PROMPT = 8;

    // GEMV modes of gl3_op_gemv
    public static final int GEMV_STORE = 0;
    public static final int GEMV_RESIDUAL = 1;
    public static final int GEMV_SWIGLU = 2;

    public static final long NOALLOC_SCRATCH_BYTES = 1280L << 10;

    /** struct gl3_config: 11 int32, 2 float, 1 uint32 (56 bytes, no padding). */
    public static final StructLayout CONFIG = MemoryLayout.structLayout(
            JAVA_INT.withName("abi_version"),
            JAVA_INT.withName("model_type"),
            JAVA_INT.withName("weight_type"),
            JAVA_INT.withName("dim"),
            JAVA_INT.withName("hidden_dim"),
            JAVA_INT.withName("n_layers"),
            JAVA_INT.withName("n_heads"),
            JAVA_INT.withName("n_kv_heads"),
            JAVA_INT.withName("head_dim"),
            JAVA_INT.withName("vocab_size"),
            JAVA_INT.withName("context_length"),
            JAVA_FLOAT.withName("rms_norm_eps"),
            JAVA_FLOAT.withName("rope_theta"),
            JAVA_INT.withName("flags"));

    /** Byte offset of a gl3_config field. */
    public static long configOffset(String field) {
        return CONFIG.byteOffset(groupElement(field));
    }

    private static final Linker LINKER = Linker.nativeLinker();
    private static final SymbolLookup LIB =
            SymbolLookup.libraryLookup(System.getProperty("gl3.library", "libgpullama3_hip.so"), Arena.global());

    private static MethodHandle fn(String name, FunctionDescriptor d) {
        return LINKER.downcallHandle(LIB.find(name).orElseThrow(() -> new UnsatisfiedLinkError(name)), d);
    }

    // ---- plan life cycle (TornadoVMMasterPlan.java:37-79, 180-202)
    public static final MethodHandle gl3_create = fn("gl3_create",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS));
    public static final MethodHandle gl3_upload = fn("gl3_upload",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, ADDRESS, JAVA_LONG, JAVA_INT));
    public static final MethodHandle gl3_set_rope_tables = fn("gl3_set_rope_tables",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT));
    public static final MethodHandle gl3_prepare = fn("gl3_prepare",
            FunctionDescriptor.of(JAVA_INT, ADDRESS));
    public static final MethodHandle gl3_destroy = fn("gl3_destroy",
            FunctionDescriptor.ofVoid(ADDRESS));

    // ---- decode (TornadoVMMasterPlan.java:127-153) and generation (InferenceEngine.java:88-131, 309-355)
    public static final MethodHandle gl3_forward = fn("gl3_forward",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, ADDRESS, ADDRESS));
    public static final MethodHandle gl3_generate_greedy = fn("gl3_generate_greedy",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS));
    public static final MethodHandle gl3_prefill = fn("gl3_prefill",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT));
    public static final MethodHandle gl3_generate_from_prompt = fn("gl3_generate_from_prompt",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS));
    public static final MethodHandle gl3_generate_sampled = fn("gl3_generate_sampled",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_FLOAT, JAVA_FLOAT,
                    ADDRESS, ADDRESS));
    public static final MethodHandle gl3_reset = fn("gl3_reset",
            FunctionDescriptor.of(JAVA_INT, ADDRESS));

    // ---- KV cache access and measurement aids
    public static final MethodHandle gl3_write_kv = fn("gl3_write_kv",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS, ADDRESS));
    public static final MethodHandle gl3_read_kv = fn("gl3_read_kv",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS, ADDRESS));
    public static final MethodHandle gl3_fill_kv_normal = fn("gl3_fill_kv_normal",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_LONG, JAVA_INT));
    public static final MethodHandle gl3_get_timing = fn("gl3_get_timing",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, ADDRESS, ADDRESS));
    public static final MethodHandle gl3_get_phase_trace = fn("gl3_get_phase_trace",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, JAVA_INT, ADDRESS));
    public static final MethodHandle gl3_get_phase_stamps = fn("gl3_get_phase_stamps",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, JAVA_LONG, ADDRESS, ADDRESS));
    public static final MethodHandle gl3_time_attention = fn("gl3_time_attention",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS));

    // ---- GGUF (ModelLoader.java:45-92)
    public static final MethodHandle gl3_gguf_config = fn("gl3_gguf_config",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, ADDRESS));
    public static final MethodHandle gl3_create_from_gguf = fn("gl3_create_from_gguf",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, ADDRESS));

    // ---- diagnostics and single-kernel entry points
    public static final MethodHandle gl3_last_error = fn("gl3_last_error",
            FunctionDescriptor.of(ADDRESS));
    public static final MethodHandle gl3_device_name = fn("gl3_device_name",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_LONG));
    public static final MethodHandle gl3_op_dequant_q8_0 = fn("gl3_op_dequant_q8_0",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_LONG, ADDRESS));
    public static final MethodHandle gl3_op_f16_to_f32 = fn("gl3_op_f16_to_f32",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_LONG, ADDRESS));
    public static final MethodHandle gl3_op_gemv = fn("gl3_op_gemv",
            FunctionDescriptor.of(JAVA_INT, JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, ADDRESS, ADDRESS, JAVA_FLOAT,
                    JAVA_INT, ADDRESS));
    public static final MethodHandle gl3_op_sample = fn("gl3_op_sample",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_FLOAT, JAVA_FLOAT, ADDRESS, JAVA_INT, ADDRESS));
    public static final MethodHandle gl3_op_attention = fn("gl3_op_attention",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT,
                    ADDRESS));
    public static final MethodHandle gl3_op_attention_noalloc = fn("gl3_op_attention_noalloc",
            FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT,
                    JAVA_INT, ADDRESS, ADDRESS));

    /** The library's message for the last failure on this thread. */
    public static String lastError() {
        try {
            MemorySegment p = (MemorySegment) gl3_last_error.invokeExact();
            return p.equals(MemorySegment.NULL) ? "" : p.reinterpret(4096).getUtf8String(0);
        } catch (Throwable t) {
            return "";
        }
    }

    /** Raises the exception the reference raises for the condition a status reports. */
    public static void check(int status) {
        if (status == OK) {
            return;
        }
        String msg = "gl3 status " + status + ": " + lastError();
        switch (status) {
            case ERR_INVALID_ARGUMENT -> throw new IllegalArgumentException(msg);
            case ERR_UNSUPPORTED -> throw new UnsupportedOperationException(msg);
            case ERR_OUT_OF_MEMORY -> throw new OutOfMemoryError(msg);
            default -> throw new IllegalStateException(msg);
        }
    }

    /** Rethrows what a downcall raised: runtime exceptions and errors as they are, the rest wrapped. */
    public static RuntimeException rethrow(Throwable t) {
        if (t instanceof RuntimeException r) {
            return r;
        }
        if (t instanceof Error e) {
            throw e;
        }
        return new IllegalStateException(t);
    }
}

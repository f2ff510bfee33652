package org.beehive.gpullama3.tornadovm;

import org.beehive.gpullama3.hip.Gl3;
import org.beehive.gpullama3.inference.state.State;
import org.beehive.gpullama3.inference.weights.standard.Phi3StandardWeights;
import org.beehive.gpullama3.inference.weights.standard.Qwen3StandardWeights;
import org.beehive.gpullama3.inference.weights.standard.StandardWeights;
import org.beehive.gpullama3.model.Configuration;
import org.beehive.gpullama3.model.Model;
import org.beehive.gpullama3.tensor.GGMLType;
import org.beehive.gpullama3.tensor.standard.ArrayFloatTensor;
import org.beehive.gpullama3.tensor.standard.FloatTensor;

import java.lang.foreign.Arena;
import java.lang.foreign.MemorySegment;

import static java.lang.foreign.ValueLayout.ADDRESS;
import static java.lang.foreign.ValueLayout.JAVA_FLOAT;
import static java.lang.foreign.ValueLayout.JAVA_INT;

/**
 * The reference's GPU execution plan (tornadovm/TornadoVMMasterPlan.java), kept
 * under its name and public API so that Model, InferenceCore and
 * InferenceEngine reach it as before, with libgpullama3_hip.so on one AMD
 * Instinct MI355X underneath instead of TornadoVM task graphs:
 *
 * <ul>
 *   <li>{@link #initializeTornadoVMPlan(State, Model)} (TornadoVMMasterPlan.java:37-79)
 *       creates the device plan, uploads every weight of the model's
 *       {@link StandardWeights} straight from the mapped GGUF (Q8_0 blocks are
 *       repacked on the device) and the host's RoPE tables, and primes it;</li>
 *   <li>{@link #tornadoVMForwardExecuteLayered(int)} (:127-153) runs one decode
 *       step of the token staged in {@code state.latestToken} (the embedding
 *       row is gathered on the device) and returns the logits as a
 *       {@link FloatTensor}, which every {@code Sampler} accepts;</li>
 *   <li>{@link #forceCopyInReadOnlyDataLayered()} (:180-195) and
 *       {@link #freeTornadoExecutionPlan()} (:200-202).</li>
 * </ul>
 *
 * One generation thread drives a plan, as with the reference.
 */
public class TornadoVMMasterPlan {
    public static final boolean ENABLE_TORNADOVM_INIT_TIME =
            Boolean.parseBoolean(System.getProperty("llama.EnableTimingForTornadoVMInit", "False"));

    private final State state;
    private final Configuration config;
    private final Arena arena = Arena.ofShared();  // plan-lifetime native memory
    private final MemorySegment plan;              // gl3_plan *
    private final MemorySegment logitsOut;         // vocab floats written by gl3_forward
    private final float[] logitsHost;              // backing array of the tensor handed to the Sampler
    private final FloatTensor logits;
    private boolean freed;

    public TornadoVMMasterPlan(State state, Model model) {
        this.state = state;
        this.config = model.configuration();
        int vocab = config.vocabularySize();
        this.logitsOut = arena.allocateArray(JAVA_FLOAT, vocab);
        this.logitsHost = new float[vocab];
        this.logits = new ArrayFloatTensor(logitsHost);
        StandardWeights w = (StandardWeights) model.weights();
        MemorySegment handle;
        try (Arena tmp = Arena.ofConfined()) {
            MemorySegment cfg = tmp.allocate(Gl3.CONFIG);
            fillConfig(cfg, model, w.getWeightType());
            MemorySegment out = tmp.allocate(ADDRESS);
            Gl3.check((int) Gl3.gl3_create.invokeExact(cfg, out));
            handle = out.get(ADDRESS, 0);
        } catch (Throwable t) {
            arena.close();
            throw Gl3.rethrow(t);
        }
        this.plan = handle;
        try {
            uploadWeights(model, w);
        } catch (RuntimeException | Error e) {
            freeTornadoExecutionPlan();
            throw e;
        }
    }

    /** Creates the plan, uploads the weights and primes it; sets it on the model. */
    public static TornadoVMMasterPlan initializeTornadoVMPlan(State state, Model model) {
        long start = System.nanoTime();
        TornadoVMMasterPlan p = new TornadoVMMasterPlan(state, model);
        long created = System.nanoTime();
        p.forceCopyInReadOnlyDataLayered();
        if (ENABLE_TORNADOVM_INIT_TIME) {
            System.err.printf("HIP plan creation and weight upload: %.2f ms%n", (created - start) / 1e6);
            System.err.printf("HIP schedule preparation: %.2f ms%n", (System.nanoTime() - created) / 1e6);
        }
        model.setTornadoVMPlan(p);
        return p;
    }

    /**
     * One decode step at {@code position} of the token in {@code state.latestToken}
     * (InferenceCore.forwardTornadoVM stages it there); the logits come back in
     * a FloatTensor that the next call overwrites.
     */
    public FloatTensor tornadoVMForwardExecuteLayered(int position) {
        try {
            Gl3.check((int) Gl3.gl3_forward.invokeExact(plan, state.latestToken, position, logitsOut,
                    MemorySegment.NULL));
        } catch (Throwable t) {
            throw Gl3.rethrow(t);
        }
        MemorySegment.copy(logitsOut, JAVA_FLOAT, 0, logitsHost, 0, logitsHost.length);
        return logits;
    }

    /** Builds the per-token schedule (idempotent; the first forward would do it too). */
    public void forceCopyInReadOnlyDataLayered() {
        try {
            Gl3.check((int) Gl3.gl3_prepare.invokeExact(plan));
        } catch (Throwable t) {
            throw Gl3.rethrow(t);
        }
    }

    /** Releases the device plan (weights, KV cache, schedule). */
    public void freeTornadoExecutionPlan() {
        if (freed) {
            return;
        }
        freed = true;
        try {
            Gl3.gl3_destroy.invokeExact(plan);
        } catch (Throwable ignored) {
            // the plan is gone either way
        }
        arena.close();
    }

    // ---------------------------------------------------------------- prompt and device-side loops

    /**
     * Forwards tokens[from, to) at positions position.. through the batched
     * prefill: their K and V land in the cache and no logits are produced (the
     * prompt phase of InferenceEngine.java:88-131, whose logits are unused).
     */
    public void prefill(int[] tokens, int from, int to, int position) {
        if (to <= from) {
            return;
        }
        try (Arena tmp = Arena.ofConfined()) {
            MemorySegment t = tmp.allocateArray(JAVA_INT, to - from);
            MemorySegment.copy(tokens, from, t, JAVA_INT, 0, to - from);
            Gl3.check((int) Gl3.gl3_prefill.invokeExact(plan, t, to - from, position));
        } catch (Throwable e) {
            throw Gl3.rethrow(e);
        }
    }

    /**
     * Forwards prompt[0, nPrompt) from {@code position} (all but the last token
     * batched), then samples nGen tokens on the device: argmax when temperature
     * is 0, else the reference's temperature / softmax / categorical or top-p
     * sampler with coins[k] as the draw of token k.  Returns the tokens.
     */
    public int[] generateSampled(int[] prompt, int nPrompt, int position, int nGen, float temperature, float topp,
                                 float[] coins) {
        try (Arena tmp = Arena.ofConfined()) {
            MemorySegment pr = tmp.allocateArray(JAVA_INT, nPrompt);
            MemorySegment.copy(prompt, 0, pr, JAVA_INT, 0, nPrompt);
            MemorySegment c = tmp.allocateArray(JAVA_FLOAT, nGen);
            MemorySegment.copy(coins, 0, c, JAVA_FLOAT, 0, nGen);
            MemorySegment out = tmp.allocateArray(JAVA_INT, nGen);
            Gl3.check((int) Gl3.gl3_generate_sampled.invokeExact(plan, pr, nPrompt, position, nGen, temperature, topp,
                    c, out));
            return out.toArray(JAVA_INT);
        } catch (Throwable e) {
            throw Gl3.rethrow(e);
        }
    }

    /** Zeroes the device KV cache (a fresh State). */
    public void reset() {
        try {
            Gl3.check((int) Gl3.gl3_reset.invokeExact(plan));
        } catch (Throwable e) {
            throw Gl3.rethrow(e);
        }
    }

    // ---------------------------------------------------------------- plan construction

    private static int modelType(Model model) {
        return switch (model.getModelType()) {
            case LLAMA_3 -> Gl3.MODEL_LLAMA_3;
            case MISTRAL -> Gl3.MODEL_MISTRAL;
            case QWEN_3 -> Gl3.MODEL_QWEN_3;
            case PHI_3 -> Gl3.MODEL_PHI_3;
            case QWEN_2 -> Gl3.MODEL_QWEN_2;                       // rejected by gl3_create (QKV bias)
            case DEEPSEEK_R1_DISTILL_QWEN -> Gl3.MODEL_DEEPSEEK_R1_DISTILL_QWEN;
            default -> -1;                                         // rejected by gl3_create
        };
    }

    private void fillConfig(MemorySegment cfg, Model model, GGMLType weightType) {
        int type = modelType(model);
        // head_dim: numberOfHeadsKey() for Qwen3 (headSize() throws there), dim / heads otherwise
        int headDim = type == Gl3.MODEL_QWEN_3 ? config.numberOfHeadsKey() : config.dim() / config.numberOfHeads();
        cfg.set(JAVA_INT, Gl3.configOffset("abi_version"), Gl3.ABI_VERSION);
        cfg.set(JAVA_INT, Gl3.configOffset("model_type"), type);
        cfg.set(JAVA_INT, Gl3.configOffset("weight_type"), weightType.ordinal());
        cfg.set(JAVA_INT, Gl3.configOffset("dim"), config.dim());
        cfg.set(JAVA_INT, Gl3.configOffset("hidden_dim"), config.hiddenDim());
        cfg.set(JAVA_INT, Gl3.configOffset("n_layers"), config.numberOfLayers());
        cfg.set(JAVA_INT, Gl3.configOffset("n_heads"), config.numberOfHeads());
        cfg.set(JAVA_INT, Gl3.configOffset("n_kv_heads"), config.numberOfKeyValueHeads());
        cfg.set(JAVA_INT, Gl3.configOffset("head_dim"), headDim);
        cfg.set(JAVA_INT, Gl3.configOffset("vocab_size"), config.vocabularySize());
        cfg.set(JAVA_INT, Gl3.configOffset("context_length"), config.contextLength());
        cfg.set(JAVA_FLOAT, Gl3.configOffset("rms_norm_eps"), config.rmsNormEps());
        cfg.set(JAVA_FLOAT, Gl3.configOffset("rope_theta"), config.ropeTheta());
        cfg.set(JAVA_INT, Gl3.configOffset("flags"), Integer.getInteger("gl3.flags", 0));
    }

    private void uploadWeights(Model model, StandardWeights w) {
        upload(Gl3.TOKEN_EMBD, 0, w.token_embedding_table);
        upload(Gl3.OUTPUT_NORM, 0, w.rms_final_weight);
        // a tied classifier is the embedding table itself: the plan uses it without a second copy
        MemorySegment cls = w.wcls.asMemorySegment(), emb = w.token_embedding_table.asMemorySegment();
        boolean tied = cls != null && emb != null && cls.address() == emb.address();
        if (!tied) {
            upload(Gl3.OUTPUT, 0, w.wcls);
        }
        for (int l = 0; l < config.numberOfLayers(); l++) {
            upload(Gl3.ATTN_NORM, l, w.rms_att_weight[l]);
            upload(Gl3.ATTN_OUTPUT, l, w.wo[l]);
            upload(Gl3.FFN_NORM, l, w.rms_ffn_weight[l]);
            if (w instanceof Phi3StandardWeights p) {
                upload(Gl3.ATTN_QKV, l, p.wqkv[l]);
                upload(Gl3.FFN_UP, l, p.wGateUp[l]);   // fused [2 * hidden][dim], gate rows first
                upload(Gl3.FFN_DOWN, l, p.wDown[l]);
            } else {
                upload(Gl3.ATTN_Q, l, w.wq[l]);
                upload(Gl3.ATTN_K, l, w.wk[l]);
                upload(Gl3.ATTN_V, l, w.wv[l]);
                upload(Gl3.FFN_GATE, l, w.w1[l]);
                upload(Gl3.FFN_DOWN, l, w.w2[l]);
                upload(Gl3.FFN_UP, l, w.w3[l]);
                if (w instanceof Qwen3StandardWeights q) {
                    upload(Gl3.ATTN_Q_NORM, l, q.attnQNorm[l]);
                    upload(Gl3.ATTN_K_NORM, l, q.attnKNorm[l]);
                }
            }
        }
        setRopeTables(w.freq_cis_real, w.freq_cis_imag);
    }

    /**
     * One tensor in its GGUF encoding.  F16 and Q8_0 tensors pass their mapped
     * slice; F32 tensors (norm weights: FP32FloatTensor exposes no segment) are
     * staged as floats for the call.
     */
    private void upload(int kind, int layer, FloatTensor t) {
        GGMLType type = t.type();
        MemorySegment seg = t.asMemorySegment();
        try (Arena tmp = Arena.ofConfined()) {
            if (type == GGMLType.F32 || seg == null || !seg.isNative()) {
                MemorySegment f = tmp.allocateArray(JAVA_FLOAT, t.size());
                for (int i = 0; i < t.size(); i++) {
                    f.setAtIndex(JAVA_FLOAT, i, t.getFloat(i));
                }
                seg = f;
                type = GGMLType.F32;
            }
            Gl3.check((int) Gl3.gl3_upload.invokeExact(plan, kind, layer, seg, seg.byteSize(), type.ordinal()));
        } catch (Throwable e) {
            throw Gl3.rethrow(e);
        }
    }

    /** The host's RoPE.precomputeFreqsCis tables ([context][head_dim / 2] each), so both paths rotate alike. */
    private void setRopeTables(FloatTensor real, FloatTensor imag) {
        int n = real.size();
        int half = n / config.contextLength();
        try (Arena tmp = Arena.ofConfined()) {
            MemorySegment c = tmp.allocateArray(JAVA_FLOAT, n);
            MemorySegment s = tmp.allocateArray(JAVA_FLOAT, n);
            for (int i = 0; i < n; i++) {
                c.setAtIndex(JAVA_FLOAT, i, real.getFloat(i));
                s.setAtIndex(JAVA_FLOAT, i, imag.getFloat(i));
            }
            Gl3.check((int) Gl3.gl3_set_rope_tables.invokeExact(plan, c, s, config.contextLength(), half));
        } catch (Throwable e) {
            throw Gl3.rethrow(e);
        }
    }
}

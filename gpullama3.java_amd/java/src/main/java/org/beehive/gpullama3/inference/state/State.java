package org.beehive.gpullama3.inference.state;

import org.beehive.gpullama3.model.Configuration;
import org.beehive.gpullama3.tensor.standard.FloatTensor;

/**
 * Per-sequence inference state, the reference's State
 * (inference/state/State.java) without its TornadoVM members: the FloatArray
 * wrappers of every activation, the flat KV caches, the position holder and the
 * reduction scratch (State.java:46-64 and their StateFields).  On the HIP path
 * the activations and the fp16 KV cache live in the device plan, the position
 * and token are arguments of each step, and the logits come back as a
 * FloatTensor, so the state keeps only what the CPU forward uses.  The model
 * states (LlamaState, Qwen2State, Qwen3State, Phi3State) fill the same
 * StateFields minus the wrapper assignments.
 */
public abstract class State {

    public final FloatTensor x;       // activation at the current position (dim)
    public final FloatTensor xb;      // same, inside a residual branch
    public final FloatTensor xb2;     // a second branch buffer (dim)
    public final FloatTensor hb;      // feed-forward hidden buffer (hidden_dim)
    public final FloatTensor hb2;     // a second hidden buffer (hidden_dim)
    public final FloatTensor q;       // query
    public final FloatTensor k;       // key
    public final FloatTensor v;       // value
    public final FloatTensor att;     // attention scores (n_heads, context)
    public final FloatTensor logits;  // output logits of the CPU forward
    public final int batchsize;

    public final FloatTensor[] keyCache;    // CPU forward's cache (n_layers, context, kv_dim)
    public final FloatTensor[] valueCache;

    public int localSize;
    /** The most recent token: the input of the next step (the HIP plan reads it in tornadoVMForwardExecuteLayered). */
    public int latestToken;

    protected State(Configuration config, int batchsize) {
        this.batchsize = -1;
        this.latestToken = -1;
        this.localSize = 256;
        StateFields f = createStateFields(config);
        this.x = f.x;
        this.xb = f.xb;
        this.xb2 = f.xb2;
        this.hb = f.hb;
        this.hb2 = f.hb2;
        this.q = f.q;
        this.k = f.k;
        this.v = f.v;
        this.att = f.att;
        this.logits = f.logits;
        this.keyCache = f.keyCache;
        this.valueCache = f.valueCache;
    }

    /** Each model state allocates its buffers with its own sizes. */
    protected abstract StateFields createStateFields(Configuration config);

    /** The buffers a model state allocates. */
    protected static class StateFields {
        public FloatTensor x, xb, xb2, hb, hb2, q, k, v, att, logits;
        public FloatTensor[] keyCache, valueCache;
    }

    @Override
    public State clone() throws CloneNotSupportedException {
        return (State) super.clone();
    }
}

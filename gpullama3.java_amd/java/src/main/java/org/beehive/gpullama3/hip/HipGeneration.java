package org.beehive.gpullama3.hip;

import org.beehive.gpullama3.auxiliary.LastRunMetrics;
import org.beehive.gpullama3.inference.InferenceCore;
import org.beehive.gpullama3.inference.sampler.Sampler;
import org.beehive.gpullama3.inference.state.State;
import org.beehive.gpullama3.model.Model;
import org.beehive.gpullama3.tensor.standard.FloatTensor;
import org.beehive.gpullama3.tokenizer.Tokenizer;
import org.beehive.gpullama3.tornadovm.TornadoVMMasterPlan;

import java.util.ArrayList;
import java.util.List;
import java.util.Set;
import java.util.function.IntConsumer;
import java.util.random.RandomGenerator;
import java.util.random.RandomGeneratorFactory;

/**
 * The GPU generation loops of InferenceEngine (generateTokensGPULlama,
 * inference/InferenceEngine.java:278-366, and its Qwen3 and Phi-3 twins at
 * :368-458 and :460-533) over the HIP
 * plan.  The loop is the reference's: the state's last token, then the prompt
 * tokens, are forwarded one position at a time; once the prompt is consumed
 * each step's logits are sampled and the sample is forwarded next, until a stop
 * token or the position limit.  What differs is how the positions whose logits
 * the loop never reads (the state's token and all prompt tokens but the last)
 * are run: as one batched prefill.
 *
 * <p>{@link #generateTokensOnDevice} goes further for the reference's own
 * samplers (argmax, or temperature + categorical / top-p with a seeded
 * generator, Sampler.selectSampler, inference/sampler/Sampler.java:74-122): the
 * sampler runs on the device after every step, and tokens come back in chunks.
 */
public final class HipGeneration {
    private HipGeneration() {
    }

    /** Tokens sampled on the device per call when streaming from the device loop. */
    static final int CHUNK = 16;

    public static List<Integer> generateTokensGPU(Model model, State state, int startPosition, List<Integer> promptTokens,
                                                  Set<Integer> stopTokens, int maxTokens, Sampler sampler, boolean echo,
                                                  IntConsumer onTokenGenerated, TornadoVMMasterPlan plan) {
        long startNanos = System.nanoTime();
        int ctx = model.configuration().contextLength();
        int limit = Math.min(maxTokens > 0 ? maxTokens : ctx, ctx);
        List<Integer> generated = new ArrayList<>();

        // the inputs in order: the state's last token, then the prompt
        int[] seq = new int[promptTokens.size() + 1];
        seq[0] = state.latestToken;
        for (int i = 0; i < promptTokens.size(); i++) {
            seq[i + 1] = promptTokens.get(i);
        }
        int pos = startPosition;
        // every input but the last prompt token only fills the cache: one prefill
        int nPrefill = Math.max(0, Math.min(seq.length - 1, limit - pos));
        plan.prefill(seq, 0, nPrefill, pos);
        if (echo) {
            for (int i = 0; i < nPrefill; i++) {
                System.err.print(Tokenizer.replaceControlCharacters(model.tokenizer().decode(List.of(seq[i + 1]))));
            }
        }
        pos += nPrefill;
        int promptIndex = nPrefill;
        int current = seq[nPrefill];

        while (pos < limit) {
            FloatTensor logits = InferenceCore.forwardTornadoVM(model, state, current, pos, plan);
            int next;
            if (promptIndex < promptTokens.size()) {
                next = promptTokens.get(promptIndex++);
                if (echo) {
                    System.err.print(Tokenizer.replaceControlCharacters(model.tokenizer().decode(List.of(next))));
                }
            } else {
                next = sampler.sampleToken(logits);
                if (onTokenGenerated != null) {
                    onTokenGenerated.accept(next);
                }
                if (echo && onTokenGenerated == null) {
                    System.err.print(Tokenizer.replaceControlCharacters(model.tokenizer().decode(List.of(next))));
                }
                generated.add(next);
                if (stopTokens.contains(next)) {
                    break;
                }
            }
            current = next;
            state.latestToken = current;
            pos++;
        }
        LastRunMetrics.setMetrics(promptIndex + generated.size(), (System.nanoTime() - startNanos) / 1e9);
        return generated;
    }

    /**
     * The same loop with the reference's sampler run on the device: temperature
     * 0 is argmax (Sampler.TENSOR_ARGMAX); otherwise the logits are divided by
     * the temperature and softmaxed, then CategoricalSampler (topp outside
     * (0, 1)) or ToppSampler draws with rng.nextFloat(1f) of a generator seeded
     * as Sampler.selectSampler seeds it, one draw per sampled token.
     */
    public static List<Integer> generateTokensOnDevice(Model model, State state, int startPosition,
                                                       List<Integer> promptTokens, Set<Integer> stopTokens,
                                                       int maxTokens, float temperature, float topp, long rngSeed,
                                                       IntConsumer onTokenGenerated, TornadoVMMasterPlan plan) {
        long startNanos = System.nanoTime();
        int ctx = model.configuration().contextLength();
        int limit = Math.min(maxTokens > 0 ? maxTokens : ctx, ctx);
        RandomGenerator rng = temperature == 0.0f ? null : RandomGeneratorFactory.getDefault().create(rngSeed);
        List<Integer> generated = new ArrayList<>();

        int[] seq = new int[promptTokens.size() + 1];
        seq[0] = state.latestToken;
        for (int i = 0; i < promptTokens.size(); i++) {
            seq[i + 1] = promptTokens.get(i);
        }
        // forwards available: positions startPosition .. limit - 1; the first sample follows the last prompt token
        int steps = limit - startPosition;
        if (steps <= promptTokens.size()) {
            // the prompt alone reaches the limit: nothing is sampled
            plan.prefill(seq, 0, Math.max(0, steps), startPosition);
            LastRunMetrics.setMetrics(Math.max(0, steps), (System.nanoTime() - startNanos) / 1e9);
            return generated;
        }
        int[] prompt = seq;
        int nPrompt = seq.length;
        int pos = startPosition;
        int budget = steps - promptTokens.size();  // tokens that may be sampled
        boolean stopped = false;
        while (budget > 0 && !stopped) {
            int n = Math.min(CHUNK, budget);
            float[] coins = new float[n];
            for (int k = 0; k < n; k++) {
                coins[k] = rng == null ? 0.0f : rng.nextFloat(1f);
            }
            int[] toks = plan.generateSampled(prompt, nPrompt, pos, n, temperature, topp, coins);
            pos += nPrompt;  // the forwarded prompt and the samples but the last now sit in the cache
            pos += n - 1;
            for (int t : toks) {
                generated.add(t);
                if (onTokenGenerated != null) {
                    onTokenGenerated.accept(t);
                }
                if (stopTokens.contains(t)) {
                    stopped = true;
                    break;
                }
            }
            budget -= n;
            // the next call forwards the last sample first
            prompt = new int[] {toks[n - 1]};
            nPrompt = 1;
            state.latestToken = toks[n - 1];
        }
        LastRunMetrics.setMetrics(promptTokens.size() + generated.size(), (System.nanoTime() - startNanos) / 1e9);
        return generated;
    }
}

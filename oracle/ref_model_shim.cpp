// ref_model_shim.cpp — C entry point into the reference's own DenseModel
// (src/model.cpp, src/transformer.cpp, src/kv_cache.cpp), compiled from the
// reference sources by oracle/Makefile into _ref/libref_model.so with no AVX2
// flags, so Attention::forward takes its scalar branch (softmax with
// std::exp, src/transformer.cpp:277-290).
//
// TEST INFRASTRUCTURE ONLY: writes golden vectors (tests/golden/make_golden.py)
// that pin the composition of the CPU decoder restatement (oracle/decoder.c).
#include <cstring>

#include "oil/kv_cache.h"
#include "oil/model.h"

using namespace oil;

extern "C" {

// cfg = {vocab, hidden, layers, heads, head_dim, ffn, max_seq}.  Weights as
// the reference holds them: emb [vocab][hidden]; per layer l, w[l*9 + i] for
// i = attn_norm, ffn_norm, q, k, v, o, gate, up, down, each Linear weight
// input-major ([in][out], the memory Linear::forward hands scalar_gemm).
// Feeds ids one token per forward call through one KVCache (the Generator's
// decode loop, src/generator.cpp:46-61) and writes every step's logits.
void ref_dense_model_run(const int64_t* cfg, float eps, float theta, const float* emb, const float* const* w,
                         const float* final_norm, const float* lm_head, const int32_t* ids, int64_t n,
                         float* logits) {
    TransformerConfig c;
    c.vocab_size = cfg[0];
    c.hidden_size = cfg[1];
    c.num_layers = cfg[2];
    c.num_heads = cfg[3];
    c.head_dim = cfg[4];
    c.ffn_hidden_size = cfg[5];
    c.max_seq_len = cfg[6];
    c.norm_eps = eps;
    c.rope_theta = theta;
    DenseModel m(c);
    auto put = [](Tensor& t, const float* src) { std::memcpy(t.data(), src, (size_t)t.numel() * 4); };
    put(m.tok_embeddings->weight, emb);
    for (int64_t l = 0; l < c.num_layers; l++) {
        auto& b = *m.layers[(size_t)l];
        const float* const* lw = w + l * 9;
        put(b.attention_norm.weight, lw[0]);
        put(b.ffn_norm.weight, lw[1]);
        put(b.attention.q_proj.weight, lw[2]);
        put(b.attention.k_proj.weight, lw[3]);
        put(b.attention.v_proj.weight, lw[4]);
        put(b.attention.o_proj.weight, lw[5]);
        put(b.ffn.gate_proj.weight, lw[6]);
        put(b.ffn.up_proj.weight, lw[7]);
        put(b.ffn.down_proj.weight, lw[8]);
    }
    put(m.norm->weight, final_norm);
    put(m.lm_head->weight, lm_head);
    KVCache kv;
    kv.init((int)c.num_layers, c.max_seq_len, c.num_heads, c.head_dim);
    for (int64_t i = 0; i < n; i++) {
        Tensor in(Shape{1, 1}, DType::F32), pos(Shape{1, 1}, DType::F32);
        in.data<float>()[0] = (float)ids[i];
        pos.data<float>()[0] = (float)i;
        Tensor out = m.forward(in, pos, &kv);
        std::memcpy(logits + i * c.vocab_size, out.data(), (size_t)c.vocab_size * 4);
    }
}

}  // extern "C"

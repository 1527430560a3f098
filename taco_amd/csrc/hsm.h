// The .hsm model file: a strict reader with the accept/reject rules of the reference
// (crates/hardshell/src/hsm/{mod,header,reader,merges}.rs) and the GPT-2 model checks of
// crates/hardshell/src/gpt2/model.rs:117-343. Host side of hs_model_load.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "common.h"

namespace hs {

struct HostLinear {
    uint32_t rows = 0, cols = 0;
    const int8_t *w = nullptr;  // [rows, cols] inside HostModel::file
    std::vector<int32_t> b, m;
    uint8_t s = 0;
};

struct HostLayerNorm {
    std::vector<int16_t> g;
    std::vector<int32_t> b;
    int32_t m = 0;
    uint8_t s = 0;
};

struct HostBlock {
    HostLayerNorm ln1, ln2;
    HostLinear c_attn, c_proj, c_fc, mlp_proj;
    int32_t score_m = 0, out_m = 0;
    uint8_t score_s = 0, out_s = 0;
    bool gelu_wide = false;
    std::vector<int8_t> gelu8;    // 256 or 65,536 entries, i8 outputs
    std::vector<int16_t> gelu16;  // i16 outputs (version 2)
    uint32_t gelu_len = 0;
};

struct HostModel {
    std::vector<uint8_t> file;  // the bytes of the .hsm file
    uint8_t hash[32] = {0};
    uint32_t version = 1;
    uint32_t n_layer = 0, n_head = 0, d_model = 0, d_ff = 0, vocab = 0, n_ctx = 0, eot = 0;
    uint32_t head_dim = 0;
    uint8_t ln_k = 0, ln_j = 0, softmax_p = 0, ln_f_bits = 8, ln_beta_frac = 0;
    uint64_t ln_eps = 1;
    const int8_t *wte = nullptr;  // [vocab, d_model]
    const int8_t *wpe = nullptr;  // [n_ctx, d_model]
    std::vector<int32_t> embed_m, logit_m, pos_m;
    uint8_t embed_s = 0, logit_s = 0, pos_s = 0;
    std::vector<HostBlock> blocks;
    HostLayerNorm ln_f;
    std::vector<int32_t> attn_exp;
    std::vector<uint64_t> logits_exp;
    std::vector<uint32_t> vocab_ends;  // token i is file bytes [vocab_off + start_i, end_i)
    std::vector<uint8_t> vocab_bytes;
    std::vector<uint32_t> merges;  // the BPE merges in rank order, (left, right) id pairs
    bool is_wide() const;
};

// Parses and validates `bytes` as Model::load does. On failure fills `err` and returns false.
bool load_host_model(const uint8_t *bytes, size_t len, HostModel &out, ModelError &err);

}  // namespace hs

// kv_engine.h -- C++ engine-side mirror of the reference's KV-cache path.
//
// The reference engine exposes load_model_and_tokenizer / generate /
// reset_state / shutdown / get_last_prefill_ms (src/engine.h:69-90) and keeps
// its cache in globals of src/engine.cpp.  This module keeps those names,
// argument meanings and error behaviour (bool/int returns plus a message on
// stderr, src/engine.cpp:4040-4043), and drives the cache sites through the C
// ABI of libkvc (include/kvc.h):
//
//   load_model_and_tokenizer   cache + state allocation   src/engine.cpp:3835-3843
//   generate                   prompt truncation           :4048-4056
//                              prefix reuse                :4058-4080
//                              batched prefill (32/batch)  :2843-2929 (append :2885, attention :2892)
//                              decode loop                 :3521-3564, :4133-4151
//   reset_state                                            :4164-4176
//
// Everything outside the KV path is synthetic, because no model weights are
// available: a token's q, gate, K and V in every attention layer are N(0,1)
// values drawn from (seed, layer, token id, position), and the next token is
// drawn from the token history and a digest of the recurrent state.  A
// Gated-DeltaNet layer's state is represented by that digest, written into
// the first two words of its recurrent state on the device at every step, so
// snapshot/restore of the real state buffers decides what a resumed request
// generates.  The attention outputs of every step are kept for inspection.
#pragma once

#include <cstdint>
#include <functional>
#include <string>
#include <vector>

struct kvc_ctx;

namespace kvengine {

enum StopReason { STOP_LENGTH = 0, STOP_EOS = 1, STOP_CALLBACK = 2 };

using TokenCallback = std::function<bool(int token_id, const std::string& text)>;

struct EngineConfig {
    int max_ctx = 4096;          // context window (g_max_ctx)
    int n_attn_layers = 8;       // full-attention layers of Qwen3.5-9B
    int n_ssm_layers = 24;       // Gated-DeltaNet layers (0 = pure attention)
    int snapshot_slots = 64;     // recurrent-state snapshots kept for prefix reuse
    int64_t pool_blocks = 0;     // K/V blocks per layer; 0 = from pool_fraction
    double pool_fraction = 0.05; // share of free HBM for the K/V pools
    uint64_t seed = 1;           // synthetic projections and sampling
    bool keep_outputs = true;    // keep every step's attention outputs
    bool verbose = false;        // print the reference's progress lines
};

// Synthetic vocabulary size (Qwen tokenizer ids are < 151936).
constexpr int kVocab = 151936;
// Prompt tokens per prefill batch (PREFILL_BATCH of the reference).
constexpr int kPrefillBatch = 32;

// ---- the reference's interface (src/engine.h:69-90) ----------------------
bool load_model_and_tokenizer(const EngineConfig& cfg);
int generate(const std::vector<int>& prompt_tokens, int max_tokens, float temperature, TokenCallback cb,
             StopReason* stop_reason = nullptr);
void reset_state();
void shutdown();
double get_last_prefill_ms();

// ---- KV-path introspection (tests) -------------------------------------------
int pos();                                  // g_pos
const std::vector<int>& cached_tokens();    // g_cached_tokens
int last_prefix_len();                      // tokens reused by the last generate()
int state_restore_mismatches();             // resumed states that differ from recomputation
kvc_ctx* context();
int32_t sequence();

// One processed position: the attention output (bf16 bits, [16 q heads][256])
// of every attention layer, and which kernel produced it.
struct StepOutput {
    int pos = 0;
    bool from_prefill = false;
    std::vector<std::vector<uint16_t>> out;  // [layer][16 * 256]
};
const std::vector<StepOutput>& step_outputs();  // positions processed by the last generate()

// The synthetic projections of one token (bf16 bits), as the engine appends
// and queries them: q, gate [16][256]; k, v [4][256].
void synthetic_projection(int layer, int token, int pos, std::vector<uint16_t>& q, std::vector<uint16_t>& gate,
                          std::vector<uint16_t>& k, std::vector<uint16_t>& v);

}  // namespace kvengine

// kv_engine.h -- C++ engine-side mirror of the reference's KV-cache path.
//
// The reference engine exposes load_model_and_tokenizer / generate /
// reset_state / shutdown / get_hang_info / get_last_prefill_ms
// (src/engine.h:69-90) and keeps its cache in globals of src/engine.cpp.  This
// module keeps those names, signatures, argument meanings and error behaviour
// (bool/int returns plus a message on stderr, src/engine.cpp:4040-4043), and
// drives the cache sites through the C ABI of libkvc (include/kvc.h):
//
//   load_model_and_tokenizer   cache + state allocation   src/engine.cpp:3835-3843
//   generate                   prompt truncation           :4048-4056
//                              prefix reuse                :4058-4080
//                              batched prefill (32/batch)  :2843-2929
//                              decode loop                 :3478-3564, :4133-4151
//   reset_state                                            :4164-4176
//   get_hang_info              last op before a blocking device call, :100-101, :4182-4185
//
// Per attention layer and token the engine calls what the reference does at
// those sites: the producer + append (kvc_qkv_append: q/k RMSNorm, RoPE, K/V
// append; :3485-3525, :2846-2889), then prefill or decode attention.  Per
// Gated-DeltaNet layer it runs the layer step on the live recurrent state
// (kvc_deltanet_step; :3197-3327, :2600-2716).  Everything outside the KV path
// is synthetic, because no model weights are available: a token's projection
// rows (the attention qkv row and the DeltaNet row) are N(0,1) values drawn
// from (seed, layer, token id, position), the norm / conv / gate weights are
// seeded too, and the next token is drawn from the token history and the last
// token's layer outputs.  A resumed request therefore generates what a fresh
// one does only if the cached K/V and the restored recurrent state are exact.
//
// Sessions.  The reference serves one sequence and its server resets it per
// request (src/server.cpp:126, :194); multi-turn reuse is the chat loop's
// pattern (src/chat.cpp:117-184).  This engine keeps a table of sessions, each
// a libkvc sequence with its own token history and sampling state, over one
// context and one prefix index: generate_session() serves any of them, and a
// turn of one conversation reuses what any session has committed (blocks and
// recurrent-state snapshots).  The reference-signature generate() serves
// session 0.  The engine is single-threaded, as the reference's is (the
// server serialises requests with a mutex, src/server.cpp:20).
#pragma once

#include <cstdint>
#include <functional>
#include <string>
#include <vector>

struct kvc_ctx;

namespace kvengine {

// Same enumerators and values as the reference (src/engine.h:23): a caller
// that stores or compares the numeric value sees the same codes.
enum StopReason { STOP_EOS = 0, STOP_LENGTH = 1, STOP_CALLBACK = 2 };

using TokenCallback = std::function<bool(int token_id, const std::string& text)>;

// Engine options.  The reference reads its shapes from the GGUF and builds
// with fixed constants; this mirror takes them from set_engine_config(), which
// applies to the next load_model_and_tokenizer().
struct EngineConfig {
    int n_attn_layers = 8;       // full-attention layers of Qwen3.5-9B
    int n_ssm_layers = 24;       // Gated-DeltaNet layers (0 = pure attention)
    int max_sessions = 8;        // live sessions (libkvc sequence slots)
    int snapshot_slots = 64;     // recurrent-state snapshots kept for prefix reuse
    int64_t pool_blocks = 0;     // K/V blocks per layer; 0 = from pool_fraction
    double pool_fraction = 0.05; // share of free HBM for the K/V pools
    uint64_t seed = 0;           // synthetic weights and projections; 0 = derived from model_path
    bool keep_outputs = true;    // keep every step's layer outputs (not only their digests)
    bool verify_restore = false; // hash the recurrent state at snapshot boundaries and
                                 // check restored states against it (costly)
    bool verbose = false;        // print the reference's progress lines
};

// Synthetic vocabulary size (Qwen tokenizer ids are < 151936).
constexpr int kVocab = 151936;
// Prompt tokens per prefill batch (PREFILL_BATCH of the reference).
constexpr int kPrefillBatch = 32;

// ---- the reference's interface (src/engine.h:69-90) ----------------------
// model_path names the synthetic model: unless the engine config sets a seed,
// the seed of every synthetic weight and projection is a hash of this string,
// so one path always gives the same model.  max_ctx is the context window
// (tokens per session), as in the reference.
bool load_model_and_tokenizer(const char* model_path, int max_ctx);
int generate(const std::vector<int>& prompt_tokens, int max_tokens, float temperature, TokenCallback cb,
             StopReason* stop_reason = nullptr);
void reset_state();
void shutdown();
// Last layer and operation before a blocking device call (src/engine.cpp:100-101,
// :4182-4185).  op: 0 none, 1 attention output read (layer = attention layer),
// 2 Gated-DeltaNet output read (layer = recurrent layer), 3 recurrent-state
// read of verify_restore (layer = recurrent layer), 4 projection-row upload
// (layer = attention layer, or 1000 + recurrent layer).  The reference's op
// numbers name its Tensix reads; these name this engine's blocking HIP calls.
void get_hang_info(int& layer, int& op);
double get_last_prefill_ms();

// ---- engine options and sessions (this mirror) ------------------------------
void set_engine_config(const EngineConfig& cfg);
const EngineConfig& engine_config();
int create_session();              // a new session id, or -1 (all slots in use / not loaded)
bool release_session(int session);
bool reset_session(int session);   // reset_state() of one session
int generate_session(int session, const std::vector<int>& prompt_tokens, int max_tokens, float temperature,
                     TokenCallback cb, StopReason* stop_reason = nullptr);

// ---- KV-path introspection (tests); session 0 unless given ---------------------
int pos(int session = 0);                                // g_pos
const std::vector<int>& cached_tokens(int session = 0);  // g_cached_tokens
int last_prefix_len(int session = 0);                    // tokens reused by the session's last generate
int state_restore_mismatches();  // restored states that differ from the state hashed
                                 // when their boundary was processed (verify_restore)
int state_restore_checks();      // restored states compared
kvc_ctx* context();
int32_t sequence(int session = 0);

// One processed position: the attention output (bf16 bits, [16 q heads][256])
// of every attention layer, the Gated-DeltaNet output ([4096]) of every
// recurrent layer, and which kernels produced them.  Decode steps also keep
// the producer's q and gate rows of every attention layer.  `digest` hashes
// every layer output of the position (kept even without keep_outputs).
struct StepOutput {
    int pos = 0;
    int token = 0;
    bool from_prefill = false;
    uint64_t digest = 0;
    std::vector<std::vector<uint16_t>> out;      // [attn layer][16 * 256]
    std::vector<std::vector<uint16_t>> ssm_out;  // [ssm layer][32 * 128]
    std::vector<std::vector<uint16_t>> q, gate;  // [attn layer][16 * 256], decode steps only
};
// positions processed by the session's last generate
const std::vector<StepOutput>& step_outputs(int session = 0);

// Width of the synthetic attention projection row: [16][q | gate][256], k [4][256], v [4][256].
constexpr int kQkvRow = 16 * 2 * 256 + 2 * 4 * 256;
// The synthetic attention projection row of one token (bf16 bits) and the
// layer's q_norm / k_norm weights (fp32 [256] each), as the engine hands them
// to kvc_qkv_append.
void synthetic_qkv_row(int layer, int token, int pos, std::vector<uint16_t>& row);
void synthetic_norm_weights(int layer, std::vector<float>& q_norm, std::vector<float>& k_norm);

}  // namespace kvengine

// kvc_internal.h -- shapes, device layouts and kernel-argument blocks shared by
// the host bookkeeping (kvc_host.cpp) and the gfx950 kernels (*.hip).
//
// HBM layout of the K/V pools (one allocation per context):
//   pool[layer][kv(0=K,1=V)][block][kv_head][tok(32)][d(256)]   bf16
// so a (block, kv_head) unit is 32*256*2 = 16 KiB contiguous and a block of one
// layer is 64 KiB.  Block ids are shared by all attention layers: a sequence's
// block table maps token position p -> block table[p / 32], slot p % 32, in
// every layer's pool.  The reference keeps one contiguous fp32 array per layer
// instead (src/engine.cpp:81-84, index pos*kv_dim + kv_h*D + d at :3539).
//
// Recurrent state of a sequence slot (one contiguous region per slot):
//   [ssm_layer][ rec fp32 [v_heads][v_dim][k_dim] | conv fp32 [rows][channels] ]
// matching g_ssm_state / g_conv_state (src/engine.cpp:86-94, :3840-3843).
//
// Snapshot slot (one contiguous region per slot):
//   [ state of one sequence (as above) | kv segment [layer][kv][seg_blocks][64 KiB] ]
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace kvc {

// Kernel specialisation: Qwen3.5 full-attention shapes (model_config.h:15-17).
constexpr int kHeadDim = 256;
constexpr int kKvHeads = 4;
constexpr int kGroup = 4;  // q heads per kv head (16 / 4)
constexpr int kQHeads = kKvHeads * kGroup;
constexpr int kBlockTok = 32;
constexpr size_t kUnitBytes = (size_t)kBlockTok * kHeadDim * 2;  // 16 KiB
constexpr size_t kBlockBytes = kUnitBytes * kKvHeads;            // 64 KiB

constexpr int kMaxBatch = 64;        // seqs per kernel launch (argument block)
constexpr int kMaxChunks = 8192;     // split-K work chunks per decode launch
// split-K partial of one work item: acc [4 q heads][256] fp32 then (m, l) per
// head, padded to whole 128-B lines so no line is shared by two items
constexpr int kItemFloats = 1056;
constexpr int kMaxDParts = 2;        // output-dim parts per decode chunk
constexpr int kCounterStride = 32;   // int32s between arrival counters (one 128-B line each)
constexpr size_t kPartBytes = (size_t)kMaxChunks * kKvHeads * kItemFloats * 4;
// one arrival counter per (sequence, kv head, output-dim part, q head of the group)
constexpr size_t kCounterBytes = (size_t)kMaxBatch * kKvHeads * kMaxDParts * kGroup * kCounterStride * 4;
// Static workspace of kvc_decode_attn_static, the entry point that allocates
// nothing: a file-scope __device__ array of this many split-K items (plus the
// arrival counters) per GPU, held until the process ends.
// gather: workgroups per 32-token work item = (K or V) x kGatherQ parts
constexpr int kGatherQ = 2;
constexpr int kGatherWgsPerItem = 2 * kGatherQ;
constexpr int kStaticItems = 4096;
constexpr size_t kStaticPartBytes = (size_t)kStaticItems * kItemFloats * 4;  // 17,301,504 B (+ 256 KiB counters)
// The automatic split-K chunk keeps a launch within this many items, in both
// workspaces, so kvc_decode_attn and kvc_decode_attn_static take the same
// split whenever the caller leaves decode_chunk_blocks at 0.
constexpr int kAutoItems = kStaticItems;
constexpr int kMaxDevices = 64;
constexpr int kTableUpdatesPerLaunch = 480;

// ---- kernel argument blocks (passed by value; must stay < 4 KiB) ----------

struct TableUpdateArgs {
    int32_t* table;   // device block table [max_seqs][max_blocks]
    int32_t n;
    int32_t pad;
    int32_t index[kTableUpdatesPerLaunch];  // slot * max_blocks + block index
    int32_t block[kTableUpdatesPerLaunch];
};

struct DecodeArgs {
    const uint16_t* kpool;  // this layer's K pool base
    const uint16_t* vpool;
    const int32_t* table;
    const uint16_t* q;      // [n_seqs][Hq][D]
    const uint16_t* k_new;  // [n_seqs][Hkv][D] or null
    const uint16_t* v_new;
    const uint16_t* gate;   // [n_seqs][Hq][D] or null
    void* out;              // [n_seqs][Hq][D]
    float* part;            // split-K workspace [item][G][D + 2]
    uint32_t part_bytes;    // its size (bound of the buffer resource)
    int32_t pad0;
    int32_t* counters;      // [kMaxBatch][Hkv][kMaxDParts][G] arrival counters, kCounterStride
                            // apart (self-resetting)
    float scale_log2;       // scale * log2(e)
    int32_t out_bf16;
    int32_t table_stride;   // max blocks per seq
    int32_t n_seqs;
    int32_t chunk_blocks;   // blocks per split-K chunk
    int32_t total_chunks;   // sum over seqs
    int32_t n_items;        // total_chunks * Hkv * d_parts
    int32_t per_xcd;        // ceil(n_items / 8)
    int32_t d_parts;        // output-dim parts per (chunk, head): 1 or 2
    int32_t gate_ref;       // 1: the reference's Schraudolph gate sigmoid; 0: exact
    int32_t pad;
    // decode step with the attention producer fused in (decode_kernel<NP, 1 or 2>):
    // q, gate and the new token's k / v come from the projection rows
    const void* qkv;        // [n_seqs][kQkvRow] (layout of QkvArgs::qkv), bf16 or fp32
    const float* q_norm;    // [D]
    const float* k_norm;    // [D]
    const float* rope;      // as QkvArgs::rope
    float eps;
    int32_t rope_half;
    int32_t rope_rows;
    int32_t qkv_f32;        // 1: fp32 rows
    int32_t slot[kMaxBatch];
    int32_t kv_len[kMaxBatch];       // keys attended (new token included)
    int32_t chunk_begin[kMaxBatch + 1];
};

struct AppendArgs {
    uint16_t* kpool;
    uint16_t* vpool;
    const int32_t* table;
    const uint16_t* k;  // [n_seqs][n_tok][Hkv][D]
    const uint16_t* v;
    int32_t table_stride;
    int32_t n_seqs;
    int32_t n_tok;
    int32_t pad;
    int32_t slot[kMaxBatch];
    int32_t pos0[kMaxBatch];  // first position written
};

// attention projection row of one token: [Hq][q | gate][D], k [Hkv][D], v [Hkv][D]
constexpr int kQkvRow = kQHeads * 2 * kHeadDim + 2 * kKvHeads * kHeadDim;

struct QkvArgs {
    const void* qkv;        // [n_seqs][n_tok][kQkvRow], fp32 or bf16
    const float* q_norm;    // [D]
    const float* k_norm;    // [D]
    const float* rope;      // cos [rope_rows][rope_half], then sin [rope_rows][rope_half]
    uint16_t* kpool;
    uint16_t* vpool;
    const int32_t* table;
    uint16_t* q_out;        // [n_seqs][n_tok][Hq][D] bf16 or null
    uint16_t* gate_out;     // likewise
    float eps;
    int32_t in_bf16;
    int32_t rope_half;      // rope_dim / 2 (0 = no RoPE)
    int32_t rope_rows;      // positions in each table
    int32_t table_stride;
    int32_t n_seqs;
    int32_t n_tok;
    int32_t pad;
    int32_t slot[kMaxBatch];
    int32_t pos0[kMaxBatch];  // first position written
};

// Gated-DeltaNet shapes the step kernel is built for (model_config.h:25-31)
constexpr int kSsmVHeads = 32;
constexpr int kSsmKHeads = 16;
constexpr int kSsmDk = 128;
constexpr int kSsmDv = 128;
constexpr int kSsmConvRows = 3;
constexpr int kSsmC = 2 * kSsmKHeads * kSsmDk + kSsmVHeads * kSsmDv;  // 8192 conv channels
constexpr int kSsmProj = kSsmC + kSsmVHeads * kSsmDv + 2 * kSsmVHeads;  // 12352 per token

struct DeltaNetArgs {
    const void* proj;       // [n_seqs][n_tok][kSsmProj], fp32 or bf16
    const float* conv_w;    // [4][kSsmC] tap-major
    const float* dt_bias;   // [kSsmVHeads]
    const float* a;         // [kSsmVHeads]
    const float* norm_w;    // [kSsmDv]
    void* out;              // [n_seqs][n_tok][kSsmVHeads * kSsmDv]
    uint8_t* state;         // state pool base
    int64_t state_bytes;    // per sequence slot
    int64_t layer_off;      // byte offset of this layer's rec state inside a slot
    int64_t rec_bytes;      // conv state follows the rec state
    float eps;
    float out_scale;
    int32_t in_bf16;
    int32_t out_bf16;
    int32_t n_seqs;
    int32_t n_tok;
    int32_t ref_math;       // 1: the reference's Schraudolph SiLU / sigmoid / softplus
    int32_t pad;
    int32_t slot[kMaxBatch];
};

struct ZeroStateArgs {
    uint8_t* state;       // state pool base
    int64_t state_bytes;  // per sequence slot (multiple of 256)
    int32_t n_slots;
    int32_t pad;
    int32_t slot[kMaxBatch];
};

struct GatherArgs {
    const uint16_t* kpool;
    const uint16_t* vpool;
    const int32_t* table;
    uint16_t* k_out;
    uint16_t* v_out;
    int32_t table_stride;
    int32_t n_seqs;
    int32_t tok0;
    int32_t total_tok;
    int32_t n_items;                    // (seq, 32-token output chunk) work items
    int32_t pad;
    int32_t slot[kMaxBatch];
    int32_t out_begin[kMaxBatch + 1];   // token offsets into the packed output
    int32_t item_begin[kMaxBatch + 1];  // first work item of each sequence
};

// K/V checksums: one work unit = one (block, K|V, kv head) unit of 16 KiB.
struct ChecksumArgs {
    const uint16_t* kpool;
    const uint16_t* vpool;
    const int32_t* table;
    uint64_t* out;                       // one checksum per unit, units of all seqs back to back
    int32_t table_stride;
    int32_t n_seqs;
    int32_t n_units;
    int32_t pad;
    int32_t slot[kMaxBatch];
    int32_t kv_len[kMaxBatch];           // tokens covered
    int32_t unit_begin[kMaxBatch + 1];   // first unit of each sequence (launch-relative)
};

struct PrefillArgs {
    const uint16_t* kpool;
    const uint16_t* vpool;
    const int32_t* table;
    const uint16_t* q;     // [n_seqs][n_q][Hq][D]
    const uint16_t* gate;  // same or null
    void* out;
    float scale_log2;
    int32_t out_bf16;
    int32_t table_stride;
    int32_t n_seqs;
    int32_t n_q;
    int32_t gate_ref;           // 1: the reference's Schraudolph gate sigmoid; 0: exact
    int32_t n_groups;           // n_seqs * Hkv (sequence, kv head) groups
    int32_t pad2;
    // prefill with the producer's q side fused in (prefill_mfma_kernel<NT, 1 or 2>):
    // q and gate come from the projection rows
    const void* qkv;            // [n_seqs][n_q][kQkvRow] (layout of QkvArgs::qkv), bf16 or fp32
    const float* q_norm;        // [D]
    const float* rope;          // as QkvArgs::rope
    float eps;
    int32_t rope_half;
    int32_t rope_rows;
    int32_t qkv_f32;            // 1: fp32 rows
    int32_t slot[kMaxBatch];
    int32_t q_pos0[kMaxBatch];  // position of query row 0
    int32_t seq_order[kMaxBatch];  // batch indices, most keys first
};

// Snapshot copy: per pair, state bytes then the K/V segment.
struct SnapshotArgs {
    uint8_t* state_base;     // live state pool
    uint8_t* snap_base;      // snapshot pool
    uint8_t* pool_base;      // K/V pools (all layers)
    const int32_t* table;
    int64_t state_bytes;     // per sequence slot
    int64_t snap_bytes;      // per snapshot slot
    int64_t layer_kv_bytes;  // bytes of one (layer, kv) pool = n_blocks * 64 KiB
    int32_t n_layers;        // attention layers
    int32_t seg_blocks;      // blocks per segment
    int32_t table_stride;
    int32_t restore;         // 0 = save (live -> snap), 1 = restore
    int32_t n_pairs;
    int32_t do_state;        // copy the recurrent state part
    int32_t do_kv;           // copy the K/V segment part
    int32_t pad;
    int32_t seq_slot[kMaxBatch];
    int32_t snap_slot[kMaxBatch];
    int32_t first_block[kMaxBatch];  // block-table index of the segment start
};

// Copy whole blocks (all layers, K and V): copy-on-write of a shared block.
struct BlockCopyArgs {
    uint8_t* pool_base;
    int64_t layer_kv_bytes;
    int32_t n_layers;
    int32_t n;
    int32_t src[kMaxBatch];
    int32_t dst[kMaxBatch];
};

// ---- launchers (kvc_kernels.hip); return hipError_t as int ---------------
// Device address of this GPU's static decode workspace (split-K partials,
// then the arrival counters), looked up once per device with
// hipGetSymbolAddress and its counters zeroed then; `device` must be current.
// Returns a hipError_t.
int static_scratch(int device, float** part, int32_t** counters);

int launch_table_update(const TableUpdateArgs& a, void* stream);
int launch_decode(const DecodeArgs& a, void* stream);
int launch_append(const AppendArgs& a, void* stream);
int launch_qkv_append(const QkvArgs& a, void* stream);
int launch_deltanet(const DeltaNetArgs& a, void* stream);
int launch_zero_state(const ZeroStateArgs& a, void* stream);
int launch_gather(const GatherArgs& a, void* stream);
int launch_checksum(const ChecksumArgs& a, void* stream);
int launch_prefill(const PrefillArgs& a, void* stream);
int launch_snapshot(const SnapshotArgs& a, void* stream);
int launch_block_copy(const BlockCopyArgs& a, void* stream);
int launch_fill_normal(uint16_t* dst, int64_t n, uint64_t seed, float scale,
                       void* stream);

}  // namespace kvc

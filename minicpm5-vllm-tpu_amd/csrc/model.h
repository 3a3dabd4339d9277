// Model runner state (host side of libmk).
#pragma once

#include <hip/hip_runtime.h>

#include <vector>

#include "mk.h"

namespace mk {

// Per-linear precision + flags of a quant string (mk_jax.py:302-318).
// Precision of one linear (the quant string's base applied to it, mk_jax.py:302-318).
enum LinQ : uint8_t { LQ_BF16, LQ_I8D, LQ_I8S, LQ_F8D, LQ_F8S };
struct QuantPlan {
  LinQ mode[4];     // qkv, o, gu, down
  bool i8[4];       // 8-bit (int8 or fp8 e4m3) weights
  bool sq, lastbf16, fqkv, fmlp;
};

// Byte offsets of the packed (K-contiguous) weights inside the caller's packed buffer.
struct PackedLayout {
  size_t wqkv, sqkv, wo, wgu, sgu, wd, wlqkv, wlo, wlgu, wld, total;
};

// Byte offsets of the forward's buffers inside the caller's workspace.
struct WorkLayout {
  size_t x, xq, sx, qkv, attn, xn, h, att, part, xnl, ql, attl, xl, gul, hl, skws, skws_bytes, total;
};

struct GraphKey {
  int bs, seq;
  const void* ids;
  const void* hidden;
  const void* logits;
  const void* ws;
  bool operator==(const GraphKey& o) const {
    return bs == o.bs && seq == o.seq && ids == o.ids && hidden == o.hidden && logits == o.logits && ws == o.ws;
  }
};

// A captured forward and an event recorded on the caller's stream after its latest replay: the exec is
// destroyed only once that event has completed (HIP does not promise deferred destruction of a graph
// that is still running).
struct CachedGraph {
  GraphKey key;
  hipGraphExec_t exec;
  hipEvent_t done;
};
// Waits for the graph's latest replay, then destroys it.
void destroy_graph(CachedGraph& g);

struct Model {
  static constexpr size_t kMaxGraphs = 16;
  mk_config cfg{};
  QuantPlan q{};
  mk_weights w{};
  PackedLayout P{};
  char* packed = nullptr;
  bool use_graph = true;
  int max_chunk = 0;   // caller's cap on sequences per chunk (0: only the 4 GiB operand limit)
  bool fuse_prep = true;   // K RoPE / V^T written by the QKV projection's epilogue (else the prep kernel)
  hipStream_t cap_stream = nullptr;
  std::vector<CachedGraph> graphs;
  void drop_graphs();   // destroy_graph on every cached graph
  ~Model();
};

int parse_quant(const char* quant, QuantPlan* p);
int validate_config(const mk_config* c);
int validate_run(const mk_config& c, int bs, int seq);
int packed_layout(const mk_config* c, const QuantPlan& q, PackedLayout* L);
int workspace_layout(const Model& m, int B, int S, WorkLayout* W);
// Sequences per chunk of a (bs, S) forward: every GEMM operand of a chunk spans < 4 GiB (32-bit
// operand offsets), at most m.max_chunk when set.  The forward runs the chunks one after another with
// one workspace of chunk size (the reference's microbatching, mk_jax.py:572-605).
int chunk_seqs(const Model& m, int bs, int S);
int model_create(const mk_config* cfg, const char* quant, const mk_weights* w, void* packed, size_t packed_bytes,
                 hipStream_t st, Model** out);
// Eager forward with an event pair around every launch: per-kind kernel time (ms) and launch counts,
// indexed by MK_KERNEL_*.  Synchronizes the stream.
int model_forward_timed(Model* m, const int32_t* ids, int bs, int seq, void* hidden, float* logits, void* ws,
                        size_t ws_bytes, hipStream_t st, float* ms, int* launches);
int model_forward(Model* m, const int32_t* ids, int bs, int seq, void* hidden, float* logits, void* ws,
                  size_t ws_bytes, hipStream_t st);
// Captures and instantiates the hipGraph of (bs, seq, buffers) without running it (no-op when cached).
int model_precompile(Model* m, const int32_t* ids, int bs, int seq, void* hidden, float* logits, void* ws,
                     size_t ws_bytes);

}  // namespace mk

// Host-side interface of the decode dataflow kernel (flow.hip): the block after the router
// logits (top-k, routed gate_up and down, shared down, combine) in one launch, for slot-major
// decode batches.
#pragma once

#include "qmoe_internal.h"
#include "route_common.h"

namespace qmoe {

struct FlowLaunch {
  const uint16_t* x;          // [N][H] the block's input rows (normalised when fused)
  int N, k, H, I, Is;
  const float* logits;        // [N][ld] from the router launch, shared gate logit in column E
  int ld;
  TopkParams P;
  const void* gu_codes;       // tiled int4 gate|up [E][2I][H]
  const uint16_t* gu_sb;
  const void* dn_codes;       // tiled int4 down [E][H][I]
  const uint16_t* dn_sb;
  int glu;                    // gated activation (QMOE_ACT_*)
  float glu_alpha, glu_limit;
  const uint16_t* sh_h;       // [N][Is] shared expert's SwiGLU output, or [N][2 Is] its gate | up
                              // rows (decode_flow_split_shared), from the router launch
  const void* sh_dn;          // shared down [H][Is], tiled bf16 or int8 (sfmt)
  const uint16_t* sh_dn_sb;
  int sfmt;
  float* w;                   // workspace: [mc] routing weights, [N] shared gates
  float* sg;
  uint16_t* h;                // [mc][I]
  uint16_t* d;                // [mc][H]
  uint16_t* sh_out;           // [N][H]
  uint32_t* sync;             // decode_flow_sync_words(N * k, H) words, zero at launch
  const uint16_t* resid;      // nullable residual rows
  uint16_t* y;                // [N][H]
};

// Whether the compiled kernel covers this shape (a slot-major batch of up to 16 tokens, c1- or
// c2-like chunking).
bool decode_flow_fits(int N, int k, int E, int H, int I, int Is);
// Whether its shared-down units read the router launch's split [gate | up] rows (sh_h 2 Is wide).
bool decode_flow_split_shared(int H, int I, int Is);
int64_t decode_flow_sync_words(int64_t mc, int H);
bool decode_flow_enabled(int N);   // the process-wide mode's choice for an N-token call
int launch_decode_flow(const FlowLaunch& L, hipStream_t stream);

}  // namespace qmoe

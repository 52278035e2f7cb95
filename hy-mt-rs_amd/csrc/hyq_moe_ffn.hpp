// The MoE FFN of a HyV3 layer (Moe::forward, src/model.rs:687-726) as
// device launch sequences, shared by the decoder (hyq_dense.cpp) and the
// standalone entry points (hyq_moe_forward_d).
//
// One row (batch 1, the decode step): router logits by the f32 GEMV, route,
// the shared expert's gate/up GEMV and the chosen experts' gate/up GEMV (rows
// of the expert stacks picked by the device-resident route result), the
// shared down GEMV and the experts' down GEMV (one workgroup row per expert
// slot), then out = residual + (shared + w_0 e_0 + ...). All int8 GEMVs with
// Q8 activations, no host round trip, so a decode step stays capturable.
//
// n rows (prefill): router logits by the f32 GEMM, route into (token,
// expert, weight) pairs, the shared expert as f16-MFMA GEMMs, the experts
// through the grouped expert kernels (launch_moe), which add w * e into the
// shared output per token in ascending expert order, then the residual.
#pragma once

#include "hyq_abi.hpp"

namespace hyq {

struct MoeFfn {
    const hyq_weight *router = nullptr; // F32 [experts][hidden]
    const float *bias_d = nullptr;      // selection bias [experts], device
    const hyq_weight *gate = nullptr, *up = nullptr, *down = nullptr;    // expert stacks
    const hyq_weight *sgate = nullptr, *sup = nullptr, *sdown = nullptr; // shared expert
    int hidden = 0, experts = 0, used = 0, mid = 0, smid = 0, normalize = 0;
    float scale = 1.f;
};

// Shapes and formats (HYQ_EINVAL / HYQ_EDTYPE with a message), as
// Model::from_gguf checks them (src/model.rs:206-235) plus this library's
// limits: widths in whole 256-value groups (the int8 GEMVs), at most
// route_max_experts() experts.
int moe_ffn_check(const MoeFfn &f, int device);

// Batch-1 temporaries: router logits [E], slot experts and weights [used],
// shared SiLU row [smid], expert SiLU rows [used][mid], shared down row [H],
// expert down rows [used][H].
struct MoeRowBuf {
    float *logits;
    int *se;
    float *sw, *hs, *he, *ps, *pe;
};
size_t moe_row_bytes(const MoeFfn &f);
MoeRowBuf moe_row_carve(const MoeFfn &f, uint8_t *base);
// out = residual + Moe::forward(xn) (out alone when residual is null) for
// one normalized row xn (f32, 16-byte aligned) and its Q8 xq; trace, when
// set, gets a copy of out; q8t, when set, records the down projections'
// input stages (the shared expert's, then the slots').
int moe_ffn_row(hipStream_t st, const MoeFfn &f, const float *xn, const Q8Ref &xq,
                const MoeRowBuf &b, const float *residual, float *out, float *trace,
                Q8Trace *q8t = nullptr);

// n-row temporaries: logits [n][E], pairs [n * used], f16 rows with scales,
// the shared SiLU rows [n][smid], the FFN output [n][H], the grouped expert
// kernels' scratch.
struct MoeRowsBuf {
    float *logits, *pw, *rs, *h, *ffo;
    int *pt, *pe;
    _Float16 *xh;
    uint8_t *scratch;
    MoeLayout L;
};
size_t moe_rows_bytes(const MoeFfn &f, int n);
MoeRowsBuf moe_rows_carve(const MoeFfn &f, int n, uint8_t *base);
// The most rows one call takes (the grouped expert kernels' limits).
int moe_rows_max(const MoeFfn &f);
int moe_ffn_rows(hipStream_t st, const MoeFfn &f, const float *xn, int n, const MoeRowsBuf &b,
                 const float *residual, float *out);

} // namespace hyq

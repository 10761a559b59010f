// Grouped (mixture-of-experts) launches of the register-dequant prefill GEMM,
// for the MoE entry points in hxq_gemm.hip.
#pragma once
#include "hxq.h"

namespace hxq {
namespace pg {

struct GroupedReq {
    const void *x;
    int32_t x_dtype;          // HXQ_BF16 / HXQ_F16
    int64_t x_rows;
    const int32_t *rows;      // sorted position -> X row (NULL: identity)
    const int32_t *seg;       // expert_offsets [n_exp + 1] (device)
    int32_t n_exp;
    int64_t n_assign;
    const hxq_expert_bank *bank0, *bank1;  // bank1 NULL: one bank
    int64_t out0, out1;       // output columns [0, out0) from bank0, [out0, out0 + out1) from bank1
    int64_t in;
    int32_t group;            // affine group size (banks with group_affine)
    void *y;                  // [n_assign, out0 + out1]
    int32_t y_dtype;
};

// Whether a bank can run the register-dequant grouped kernel.
bool grouped_ok(const hxq_expert_bank *b, int64_t out, int64_t in, int32_t group);
// Launches it (errors as hxq_* return codes).
int grouped_gemm(const GroupedReq &r, hipStream_t stream);

}  // namespace pg
}  // namespace hxq

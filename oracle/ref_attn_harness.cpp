// ref_attn_harness.cpp -- C-ABI harness over the reference's SYCL attention
// kernels run on the CPU through the reference's own host shim
// (tests/host_sycl/sycl/sycl.hpp) -- TEST INFRASTRUCTURE.
//
// nova::syclk::attn_decode (src/kernel/sycl/attn.cpp:41-161) is the same split-K
// algorithm as fa_split_paged_kernel + fa_combine_kernel (src/kernel/attn.cu:163-289)
// on a contiguous [pos][NKV][HD] fp32 cache; nova::syclk::attn_prefill
// (attn.cpp:166-257) is the causal prefill.  The paged kernels claim bitwise
// equality with the contiguous ones (attn.cu:4-9), so tests gather pages
// through the block table first.  One .so per model geometry
// (-DNOVA_SYCL_MODEL_*), as the reference welds shapes at compile time.
#include <cstdint>
#include "kernels.h"

extern "C" {
void ref_attn_geom(int* nh, int* nkv, int* hd, int* max_split) {
    *nh = nova::syclk::kNH; *nkv = nova::syclk::kNKV; *hd = nova::syclk::kHD;
    *max_split = nova::syclk::kAttnSplit;
}
int ref_attn_decode_scratch_floats(void) { return nova::syclk::attn_decode_scratch_floats(); }
void ref_attn_decode(const float* q, const float* kc, const float* vc, float* o, int n_past,
                     float* scratch) {
    sycl::queue qu;
    nova::syclk::attn_decode(q, kc, vc, o, n_past, scratch, qu);
}
void ref_attn_prefill(const float* q, const float* kc, const float* vc, float* o, int n_q, int n_past) {
    sycl::queue qu;
    nova::syclk::attn_prefill(q, kc, vc, o, n_q, n_past, qu);
}
}

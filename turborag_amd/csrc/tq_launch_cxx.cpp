// The reference's C++ launchers of the turbo_prod path (C linkage, the names
// and parameters of include/tq_turbo_prod.cuh:45-101), each the matching C
// entry of turboquant.h; a failed call throws std::runtime_error with the
// entry's message, as the reference's TQ_CHECK_LAUNCH does
// (include/tq_cuda_check.h:18-24).
#include <stdexcept>
#include <string>

#include "tq_turbo_prod_launch.h"

namespace {
void check(int rc) {
    if (rc == -1) throw std::runtime_error("turbo_prod launcher: a required pointer is NULL");
    if (rc != 0) throw std::runtime_error(std::string(tq_last_error()));
}
}  // namespace

extern "C" {

TQTurboProdPageLayout make_tq_turbo_prod_page_layout(const TQConfig& cfg) {
    TQTurboProdPageLayout layout{};
    check(tq_make_turbo_prod_layout(&cfg, &layout));
    return layout;
}

void launch_tq_turbo_prod_pack_kv(const uint16_t* key, const uint16_t* value,
                                  const int32_t* slot_mapping, uint8_t* page_pool,
                                  const TQTurboProdPageLayout& layout, const TQConfig& cfg,
                                  int num_tokens, hipStream_t stream, float* debug_k_rot,
                                  float* debug_v_rot, float* debug_kn, float* debug_vn,
                                  int* debug_kidx, int* debug_vidx) {
    if (debug_k_rot || debug_v_rot || debug_kn || debug_vn || debug_kidx || debug_vidx)
        check(tq_launch_turbo_prod_pack_kv_debug(key, value, slot_mapping, page_pool, &layout, &cfg,
                                                 num_tokens, stream, debug_k_rot, debug_v_rot,
                                                 debug_kn, debug_vn, debug_kidx, debug_vidx));
    else
        check(tq_launch_turbo_prod_pack_kv(key, value, slot_mapping, page_pool, &layout, &cfg,
                                           num_tokens, stream));
}

void launch_tq_turbo_prod_dequant_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                                     uint16_t* out_key, uint16_t* out_value,
                                     const TQTurboProdPageLayout& layout, const TQConfig& cfg,
                                     int num_tokens, hipStream_t stream) {
    check(tq_launch_turbo_prod_dequant_kv(page_pool, slot_mapping, out_key, out_value, &layout,
                                          &cfg, num_tokens, stream));
}

void launch_tq_turbo_prod_fused_attention_logits(const uint16_t* query, const uint8_t* page_pool,
                                                 const int32_t* slot_mapping, float* logits,
                                                 const TQTurboProdPageLayout& layout,
                                                 const TQConfig& cfg, int num_queries,
                                                 int num_kv_tokens, hipStream_t stream) {
    check(tq_launch_turbo_prod_fused_attention_logits(query, page_pool, slot_mapping, logits,
                                                      &layout, &cfg, num_queries, num_kv_tokens,
                                                      stream));
}

void launch_tq_turbo_prod_fused_attention_output(const uint16_t* query, const uint8_t* page_pool,
                                                 const int32_t* slot_mapping, uint16_t* output,
                                                 const TQTurboProdPageLayout& layout,
                                                 const TQConfig& cfg, int num_queries,
                                                 int num_kv_tokens, hipStream_t stream) {
    check(tq_launch_turbo_prod_fused_attention_output(query, page_pool, slot_mapping, output,
                                                      &layout, &cfg, num_queries, num_kv_tokens,
                                                      stream));
}

}  // extern "C"

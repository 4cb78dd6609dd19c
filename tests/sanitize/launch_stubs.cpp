// launch_stubs.cpp — host-only stand-ins for the device launchers of
// libturboquant (the functions defined in the .hip files), so the host
// sources (tq_capi.cpp, tq_pool.cpp, tq_loader.cpp, tq_store.cpp) link into
// a CPU executable built with AddressSanitizer and UndefinedBehaviorSanitizer.
// Every stand-in throws: the sanitized build checks host validation, error
// paths and file parsing, never kernels.
#include "tq_internal.h"

namespace tq {
namespace {
[[noreturn]] void no_device(const char* what) {
    throw Error(std::string(what) + ": no device code in the sanitizer build");
}
}  // namespace

void launch_pack(Scheme, const uint16_t*, const uint16_t*, const int32_t*, uint8_t*,
                 const PageGeom&, int, hipStream_t) { no_device("pack"); }
void launch_prod_pack_debug(const uint16_t*, const uint16_t*, const int32_t*, uint8_t*,
                            const PageGeom&, int, const PackDebug&, hipStream_t) {
    no_device("pack debug");
}
void launch_dequant(Scheme, const uint8_t*, const int32_t*, uint16_t*, uint16_t*,
                    const PageGeom&, int, hipStream_t, bool) { no_device("dequant"); }
void launch_pack_layers(Scheme, const uint16_t* const*, const uint16_t* const*, const int32_t*,
                        uint8_t* const*, const PageGeom&, int, int, hipStream_t) {
    no_device("pack layers");
}
void launch_dequant_layers(Scheme, const uint8_t* const*, const int32_t*, uint16_t* const*,
                           uint16_t* const*, const PageGeom&, int, int, hipStream_t, bool) {
    no_device("dequant layers");
}
void launch_logits(const uint16_t*, const uint8_t*, const int32_t*, float*, const PageGeom&, int,
                   int, hipStream_t) { no_device("logits"); }
void launch_paged_attention(Scheme, const uint16_t*, const uint8_t*, const int32_t*, int,
                            const int32_t*, const int32_t*, uint16_t*, const PageGeom&, int, int,
                            hipStream_t) { no_device("paged attention"); }
void launch_attention(Scheme, const uint16_t*, const uint8_t*, const int32_t*, uint16_t*,
                      const PageGeom&, int, int, hipStream_t, const Scratch&) {
    no_device("attention");
}
void launch_qjl_pack(const uint16_t*, const uint16_t*, const int32_t*, uint8_t*, const QjlGeom&,
                     int, hipStream_t) { no_device("qjl pack"); }
void launch_qjl_dequant(const uint8_t*, const int32_t*, uint16_t*, uint16_t*, const QjlGeom&, int,
                        hipStream_t) { no_device("qjl dequant"); }
void launch_qjl_attention(const uint16_t*, const uint8_t*, const int32_t*, uint16_t*,
                          const QjlGeom&, int, int, hipStream_t) { no_device("qjl attention"); }
void launch_int4_pack(const uint16_t*, const uint16_t*, const int32_t*, uint8_t*, const Int4Geom&,
                      int, hipStream_t) { no_device("int4 pack"); }
void launch_int4_dequant(const uint8_t*, const int32_t*, uint16_t*, uint16_t*, const Int4Geom&,
                         int, hipStream_t) { no_device("int4 dequant"); }
void launch_dense_copy(bool, const uint16_t*, const uint16_t*, uint16_t*, uint16_t*,
                       const int32_t*, uint8_t*, const DenseGeom&, int, hipStream_t) {
    no_device("dense copy");
}
void launch_attention_ref(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*,
                          int, int, int, int, hipStream_t) { no_device("attention_ref"); }

}  // namespace tq

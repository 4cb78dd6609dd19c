// Test-infrastructure driver linked against the reference's own legacy page
// factories (src/tq_layout.cpp, src/tq_dense_layout.cpp), compiled in place
// from /root/reference by oracle/build_ref.sh.  Prints one line per config:
//   B H D align scale_fp32 | int4: code scale kc vc ks vs kcb vcb ksb vsb page | dense: elem k v kb vb page
// ("int4: -" where the reference factory throws).
#include <cstdio>
#include <stdexcept>
#include "tq_dense_layout.h"
#include "tq_layout.h"

int main() {
    const int Bs[] = {1, 8, 16, 32};
    const int Hs[] = {1, 2, 8};
    const int Ds[] = {2, 8, 64, 128};
    const int aligns[] = {1, 64, 256};
    for (int B : Bs)
        for (int H : Hs)
            for (int D : Ds)
                for (int al : aligns)
                    for (int f32 = 0; f32 < 2; ++f32) {
                        TQConfig cfg;
                        cfg.block_size = B;
                        cfg.num_kv_heads = H;
                        cfg.head_dim = D;
                        cfg.nbits = 4;
                        cfg.group_size = D;
                        cfg.page_alignment = al;
                        cfg.scale_type = f32 ? TQScaleType::FP32 : TQScaleType::FP16;
                        std::printf("%d %d %d %d %d | ", B, H, D, al, f32);
                        TQPageLayout l = make_tq_page_layout(cfg);
                        std::printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu | ",
                                    l.code_bytes_per_token_head, l.scale_bytes_per_token_head,
                                    l.k_codes_offset, l.v_codes_offset, l.k_scales_offset,
                                    l.v_scales_offset, l.k_codes_bytes, l.v_codes_bytes,
                                    l.k_scales_bytes, l.v_scales_bytes, l.page_size_bytes);
                        TQDensePageLayout d = make_tq_dense_page_layout(cfg);
                        std::printf("%zu %zu %zu %zu %zu %zu\n", d.elem_bytes, d.k_offset,
                                    d.v_offset, d.k_bytes, d.v_bytes, d.page_size_bytes);
                    }
    // configs the factory rejects
    const int bad[][2] = {{8, 128}, {4, 64}, {2, 128}};
    for (const auto& b : bad) {
        TQConfig cfg;
        cfg.nbits = b[0];
        cfg.group_size = b[1];
        cfg.head_dim = 128;
        try {
            make_tq_page_layout(cfg);
            std::printf("reject nbits=%d group=%d: accepted\n", b[0], b[1]);
        } catch (const std::exception&) {
            std::printf("reject nbits=%d group=%d: throws\n", b[0], b[1]);
        }
    }
    return 0;
}

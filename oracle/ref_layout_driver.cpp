// Test-infrastructure driver linked against the reference's own layout
// sources (src/tq_turbo_mse_layout.cpp, src/tq_layout.cpp) compiled in place
// from /root/reference by oracle/build_ref.sh.  Prints one line per config:
//   B H D nbits align | mse: code norm k v kn vn page | legacy: page
// so tests can compare the reference factories with this build's.
#include <cstdio>
#include <cstdlib>
#include "tq_turbo_mse_layout.h"
#include "tq_layout.h"

int main(int argc, char** argv) {
    const int Bs[] = {1, 8, 16, 32};
    const int Hs[] = {1, 2, 8};
    const int Ds[] = {2, 8, 64, 128};
    const int aligns[] = {1, 64, 256};
    for (int B : Bs)
        for (int H : Hs)
            for (int D : Ds)
                for (int al : aligns) {
                    TQConfig cfg;
                    cfg.block_size = B;
                    cfg.num_kv_heads = H;
                    cfg.head_dim = D;
                    cfg.nbits = 4;
                    cfg.group_size = D;
                    cfg.page_alignment = al;
                    TQTurbomsePageLayout m = make_tq_turbo_mse_page_layout(cfg);
                    TQPageLayout l = make_tq_page_layout(cfg);
                    std::printf("%d %d %d %d %d | %zu %zu %zu %zu %zu %zu %zu | %zu\n", B, H, D,
                                cfg.nbits, al, m.code_bytes_per_token_head,
                                m.norm_bytes_per_token_head, m.k_codes_offset, m.v_codes_offset,
                                m.k_norms_offset, m.v_norms_offset, m.page_size_bytes,
                                l.page_size_bytes);
                }
    return 0;
}

// Host-only driver for the weight-file readers (csrc/mnb_pack.cpp), built with
// AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_loader_sanitized.py:
// opens every file named on the command line and, for each that opens, lists
// and reads every triplet and asks for tensor infos.  The device entry points
// the reader also calls (weight upload, quantizer) are replaced by stubs that
// fail, and error reports go nowhere: only the parsing code runs.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "mnb.h"

namespace mnb {
int32_t report(int32_t code, const char *) { return code; }
}  // namespace mnb

extern "C" {
const char *mnb_last_error(void) { return ""; }
int32_t mnb_weight_create(mnb_context *, int32_t, int32_t, int32_t, int32_t, const uint8_t *, int64_t, const void *,
                          int32_t, int64_t, const uint8_t *, int64_t, int32_t, uint32_t, mnb_weight **) {
    return MNB_ERR_NO_DEVICE;
}
int32_t mnb_weight_quantize(mnb_context *, const void *, int32_t, int32_t, int32_t, int32_t, uint32_t, mnb_weight **) {
    return MNB_ERR_NO_DEVICE;
}
}

int main(int argc, char **argv) {
    int opened = 0, reads = 0;
    for (int i = 1; i < argc; ++i) {
        mnb_pack *p = nullptr;
        if (mnb_pack_open(argv[i], &p) != MNB_OK) continue;
        ++opened;
        int32_t kind = 0, n = 0;
        mnb_pack_kind(p, &kind);
        mnb_pack_weight_count(p, &n);
        char name[4096];
        int64_t len = 0;
        mnb_pack_find_projection(p, 0, "q_proj", name, sizeof name, &len);
        for (int w = 0; w < n; ++w) {
            if (mnb_pack_weight_name(p, w, name, sizeof name, &len) != MNB_OK) continue;
            int32_t dtype = 0, ndims = 0;
            int64_t dims[8];
            mnb_pack_tensor_info(p, name, &dtype, dims, 8, &ndims);
            mnb_triplet_info info;
            if (mnb_pack_weight_info(p, name, &info) != MNB_OK) continue;
            if (info.q_bytes > (1 << 28) || info.scale_count > (1 << 26) || info.zp_bytes > (1 << 26)) continue;
            std::vector<uint8_t> q(info.q_bytes > 0 ? info.q_bytes : 1), zp(info.zp_bytes > 0 ? info.zp_bytes : 1);
            std::vector<float> s(info.scale_count > 0 ? info.scale_count : 1);
            if (mnb_pack_read_weight(p, name, q.data(), info.q_bytes, s.data(), info.scale_count, zp.data(),
                                     info.zp_bytes) == MNB_OK)
                ++reads;
        }
        for (const char *t : {"model.embed_tokens.weight", "lm_head.weight", "a"}) {
            int32_t dtype = 0, ndims = 0;
            int64_t dims[8];
            mnb_pack_tensor_info(p, t, &dtype, dims, 8, &ndims);
        }
        mnb_pack_close(p);
    }
    printf("files %d opened %d reads %d\n", argc - 1, opened, reads);
    return 0;
}

// gguf_sanitize_driver.cpp -- host-only driver for tests/test_gguf_sanitize.py:
// the GGUF reader (llm_amd/csrc/q8_gguf.cpp) built alone with AddressSanitizer
// and UndefinedBehaviorSanitizer, run over every file named on the command
// line.  Each file is opened and, if it parses, every accessor is called on
// every key and tensor and every byte of every tensor view is read, so an
// access outside the mapping or the parsed tables stops the run with the
// sanitizer's report.  Prints one line per file: "ok", "parsed" or the status.
//
// The reader's two links into the rest of the library are defined here:
// q8i::set_error (the message store) and q8_weight_resident, which only
// q8_gguf_weight calls and this driver never does.
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../include/q8gguf.h"
#include "../include/q8mi.h"
#include "../llm_amd/csrc/q8_internal.h"

namespace q8i {
int set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace q8i

extern "C" int q8_weight_resident(q8_ctx *, const void *, size_t, int, int, const q8_weight **) {
    return Q8_ERR_UNSUPPORTED;
}

static unsigned read_everything(const q8_gguf *g) {
    unsigned sum = 0;  // folded from every byte read, so no read is dead
    uint32_t version;
    uint64_t alignment, data_start, file_bytes;
    if (q8_gguf_layout(g, &version, &alignment, &data_start, &file_bytes) == Q8_OK) sum += version;
    uint64_t keys = 0;
    if (q8_gguf_meta_count(g, &keys) != Q8_OK) return sum;
    for (uint64_t i = 0; i < keys; i++) {
        const char *key = nullptr;
        if (q8_gguf_meta_key_at(g, i, &key) != Q8_OK || !key) continue;
        sum += (unsigned)strlen(key);
        uint32_t type = 0, elem = 0;
        uint64_t len = 0;
        q8_gguf_meta_type(g, key, &type, &elem, &len);
        uint64_t u;
        float f;
        int b;
        const char *s;
        uint64_t slen;
        if (q8_gguf_meta_u64(g, key, &u) == Q8_OK) sum += (unsigned)u;
        if (q8_gguf_meta_f32(g, key, &f) == Q8_OK) sum += (unsigned)(f != f);
        if (q8_gguf_meta_bool(g, key, &b) == Q8_OK) sum += (unsigned)b;
        if (q8_gguf_meta_str(g, key, &s, &slen) == Q8_OK)
            for (uint64_t c = 0; c <= slen; c++) sum += (unsigned char)s[c];  // the NUL included
        q8_gguf_has_key_prefix(g, key);
        // arrays: ask for the length, then read all of it (bounded, so a
        // mutated length cannot make the driver itself allocate wildly)
        const uint64_t cap = len < (1u << 20) ? len : (1u << 20);
        std::vector<int32_t> iv(cap + 1);
        std::vector<float> fv(cap + 1);
        std::vector<const char *> sp(cap + 1);
        std::vector<uint64_t> sl(cap + 1);
        uint64_t got = 0;
        if (q8_gguf_meta_i32_array(g, key, iv.data(), cap, &got) == Q8_OK)
            for (uint64_t e = 0; e < (got < cap ? got : cap); e++) sum += (unsigned)iv[e];
        if (q8_gguf_meta_f32_array(g, key, fv.data(), cap, &got) == Q8_OK)
            for (uint64_t e = 0; e < (got < cap ? got : cap); e++) sum += (unsigned)(fv[e] != fv[e]);
        if (q8_gguf_meta_str_array(g, key, sp.data(), sl.data(), cap, &got) == Q8_OK)
            for (uint64_t e = 0; e < (got < cap ? got : cap); e++)
                for (uint64_t c = 0; c < sl[e]; c++) sum += (unsigned char)sp[e][c];
    }
    uint64_t tensors = 0;
    if (q8_gguf_tensor_count(g, &tensors) != Q8_OK) return sum;
    for (uint64_t i = 0; i < tensors; i++) {
        q8_gguf_tensor_info t;
        if (q8_gguf_tensor_at(g, i, &t) != Q8_OK) continue;
        for (uint64_t c = 0; c <= t.name_len; c++) sum += (unsigned char)t.name[c];
        for (uint32_t d = 0; d < t.n_dims; d++) sum += (unsigned)t.dims[d];
        q8_gguf_tensor_info by_name;
        if (q8_gguf_tensor(g, t.name, &by_name) == Q8_OK) sum += (unsigned)by_name.byte_len;
        for (uint64_t c = 0; c < t.byte_len; c++) sum += t.data[c];
    }
    return sum;
}

int main(int argc, char **argv) {
    unsigned total = 0;
    for (int i = 1; i < argc; i++) {
        q8_gguf *g = nullptr;
        const int rc = q8_gguf_open(argv[i], &g);
        if (rc != Q8_OK) {
            printf("%s status %d\n", argv[i], rc);
            continue;
        }
        total += read_everything(g);
        q8_gguf_close(g);
        printf("%s parsed\n", argv[i]);
    }
    printf("done %u\n", total);
    return 0;
}

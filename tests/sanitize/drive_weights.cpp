// Sanitizer driver of the library's host checkpoint readers (aarambh-ai_amd/csrc/weights.cpp),
// built with AddressSanitizer and UndefinedBehaviorSanitizer by tests/sanitize/Makefile.  It
// decodes every tensor of the committed fixtures and feeds truncated, corrupted and
// malformed files to the readers: every case must end in a status code, never in an
// out-of-bounds access.  The context entry points weights.cpp calls are not exercised
// here (they need a GPU); the definitions below only satisfy the linker.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/aarambh_hip.h"

namespace aarh {
int ctx_fail(aarh_ctx*, int code, const char*) { return code; }
int lat_ctx_fail(aarh_lat_ctx*, int code, const char*) { return code; }
int rope_scaling_check(int, int, const aarh_rope_scaling*, std::string&) { return 0; }
}  // namespace aarh
extern "C" {
int aarh_get_config(const aarh_ctx*, aarh_model_config*) { return AARH_ERR_CONFIG; }
int aarh_num_tensors(const aarh_ctx*) { return 0; }
int aarh_tensor_info(const aarh_ctx*, int, char*, int, int64_t*, int64_t*, int32_t*) { return AARH_ERR_SHAPE; }
int aarh_load_tensor_f32(aarh_ctx*, int, const float*, int64_t) { return AARH_ERR_CONFIG; }
int aarh_set_rope_scaling(aarh_ctx*, const aarh_rope_scaling*) { return AARH_ERR_CONFIG; }
int aarh_lat_get_config(const aarh_lat_ctx*, aarh_lat_config*) { return AARH_ERR_CONFIG; }
int aarh_lat_num_tensors(const aarh_lat_ctx*) { return 0; }
int aarh_lat_tensor_info(const aarh_lat_ctx*, int, char*, int, int64_t*, int64_t*, int32_t*) { return AARH_ERR_SHAPE; }
int aarh_lat_load_tensor_f32(aarh_lat_ctx*, int, const float*, int64_t) { return AARH_ERR_CONFIG; }
}

static std::vector<unsigned char> slurp(const std::string& p) {
    std::vector<unsigned char> b;
    FILE* f = fopen(p.c_str(), "rb");
    if (!f) return b;
    int ch;
    while ((ch = fgetc(f)) != EOF) b.push_back((unsigned char)ch);
    fclose(f);
    return b;
}

static void spit(const std::string& p, const std::vector<unsigned char>& b) {
    FILE* f = fopen(p.c_str(), "wb");
    if (!f) exit(2);
    if (!b.empty()) fwrite(b.data(), 1, b.size(), f);
    fclose(f);
}

static const char* NAMES[] = {"embedding.weight", "blocks.0.norm1.weight", "blocks.0.attn.wq.weight",
                              "blocks.0.mixer_conv.weight", "blocks.0.attn.dsa.index_q.weight", "edge.constant",
                              "edge.subnormal_scale", "edge.overflow", "edge.wide", "missing.tensor"};

static int read_all(const std::string& path, bool gguf) {
    int ok = 0;
    for (const char* n : NAMES) {
        int64_t numel = 0, shape[8];
        int32_t nd = 0, enc = 0;
        int st = gguf ? aarh_gguf_read_tensor(path.c_str(), n, nullptr, 0, &numel, &nd, shape, &enc)
                      : aarh_safetensors_read_tensor(path.c_str(), n, nullptr, 0, &numel, &nd, shape);
        if (st) continue;
        std::vector<float> v((size_t)numel + 1);
        st = gguf ? aarh_gguf_read_tensor(path.c_str(), n, v.data(), numel, nullptr, nullptr, nullptr, nullptr)
                  : aarh_safetensors_read_tensor(path.c_str(), n, v.data(), numel, nullptr, nullptr, nullptr);
        if (!st) ok++;
        if (numel > 0) {  // a too-small buffer is refused
            st = gguf ? aarh_gguf_read_tensor(path.c_str(), n, v.data(), numel - 1, nullptr, nullptr, nullptr, nullptr)
                      : aarh_safetensors_read_tensor(path.c_str(), n, v.data(), numel - 1, nullptr, nullptr, nullptr);
            if (st != AARH_ERR_SHAPE) {
                fprintf(stderr, "short buffer accepted for %s\n", n);
                exit(1);
            }
        }
    }
    (void)aarh_host_last_error();
    return ok;
}

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    const std::string gold = argv[1], tmp = argv[2];
    const char* files[] = {"weights_tiny_q4km.gguf", "weights_tiny_q80.gguf", "weights_tiny_f32.safetensors",
                           "weights_tiny_f16.safetensors", "weights_tiny_bf16.safetensors"};
    for (const char* f : files) {
        const bool gguf = strstr(f, ".gguf") != nullptr;
        const std::string p = gold + "/" + f;
        if (read_all(p, gguf) != 9) {
            fprintf(stderr, "%s: not every fixture tensor decoded\n", f);
            return 1;
        }
        aarh_model_config mc{};
        aarh_rope_scaling rs{};
        aarh_lat_config lc{};
        if (gguf && (aarh_gguf_config(p.c_str(), &mc) != AARH_OK || aarh_gguf_rope_scaling(p.c_str(), &rs) != AARH_OK))
            return 1;
        // every truncation and a sweep of single-byte corruptions end in a status code
        const std::vector<unsigned char> b = slurp(p);
        const std::string q = tmp + "/mut" + (gguf ? ".gguf" : ".safetensors");
        for (size_t cut = 0; cut < b.size(); cut += (cut < 256 ? 1 : 97)) {
            spit(q, std::vector<unsigned char>(b.begin(), b.begin() + cut));
            read_all(q, gguf);
            if (gguf) (void)aarh_gguf_config(q.c_str(), &mc), (void)aarh_gguf_rope_scaling(q.c_str(), &rs),
                (void)aarh_lat_gguf_config(q.c_str(), &lc);
        }
        unsigned seed = 12345;
        for (int t = 0; t < 400; t++) {
            std::vector<unsigned char> m = b;
            seed = seed * 1103515245u + 12345u;
            const size_t at = (seed >> 8) % m.size();
            seed = seed * 1103515245u + 12345u;
            m[at] = (unsigned char)(seed >> 16);
            spit(q, m);
            read_all(q, gguf);
            if (gguf) (void)aarh_gguf_config(q.c_str(), &mc), (void)aarh_gguf_rope_scaling(q.c_str(), &rs),
                (void)aarh_lat_gguf_config(q.c_str(), &lc);
        }
    }
    printf("checkpoint reader sanitizer run: ok\n");
    return 0;
}

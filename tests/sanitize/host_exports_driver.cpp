// host_exports_driver.cpp -- exercises the library's host-only code under
// AddressSanitizer and UndefinedBehaviorSanitizer on the CPU (no GPU):
// the weight-file mapping, the coloured host buffers and their copies, the
// layer coordinate, the slot manager, and the registry and error paths that
// every entry point takes when no device is visible.  Built and run by
// tests/test_host_sanitizers.py; any sanitizer report fails the run.
#include <fcntl.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "gncx_llm_core.h"

#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            std::exit(1);                                                     \
        }                                                                     \
    } while (0)

static void file_mapping(const char* dir) {
    char path[512];
    std::snprintf(path, sizeof(path), "%s/weights.bin", dir);
    std::vector<uint8_t> bytes(3 * 4096 + 123);
    for (size_t i = 0; i < bytes.size(); ++i) bytes[i] = static_cast<uint8_t>(i * 7 + 3);
    FILE* f = std::fopen(path, "wb");
    CHECK(f && std::fwrite(bytes.data(), 1, bytes.size(), f) == bytes.size());
    std::fclose(f);
    size_t size = 0;
    void* h = gncx_gla_map_readonly(path, &size);
    CHECK(h && size == bytes.size());
    const uint8_t* base = gncx_gla_get_base_ptr(h);
    CHECK(base && std::memcmp(base, bytes.data(), bytes.size()) == 0);
    gncx_gla_prefetch_range(base, 0, size);
    gncx_gla_prefetch_range(base, size - 1, 1);
    gncx_gla_prefetch_range(base, 4096, 0);
    gncx_gla_unmap(h);
    gncx_gla_unmap(nullptr);
    CHECK(gncx_gla_map_readonly("/nonexistent/weights.bin", &size) == nullptr);
    CHECK(gncx_gla_get_base_ptr(nullptr) == nullptr);
}

static void host_buffers() {
    const size_t sizes[] = {1, 64, 4096, 4097, 1 << 20, (1 << 20) + 1, 3 << 20, 65 << 20};
    std::vector<void*> hs;
    for (size_t sz : sizes)
        for (uint8_t k = 0; k < 3; ++k) {
            void* h = gncx_ram_alloc_colored(sz, k, static_cast<uint8_t>(k * 3 + 1), static_cast<uint8_t>(k + 2));
            CHECK(h);
            uint8_t* p = gncx_ram_get_ptr(h);
            CHECK(p);
            std::memset(p, 0x5a, sz);  // the whole range is the caller's
            CHECK(gncx_ram_get_ddr3_bank(h) < 8 && gncx_ram_get_l1_set(h) < 64);
            hs.push_back(h);
        }
    for (int i = 0; i < 5; ++i) {
        void* h = gncx_ram_alloc(static_cast<size_t>(1000 + 333 * i));
        CHECK(h && gncx_ram_get_ptr(h));
        hs.push_back(h);
    }
    // copies at the edges of a buffer
    std::vector<uint8_t> src(10000);
    for (size_t i = 0; i < src.size(); ++i) src[i] = static_cast<uint8_t>(i);
    void* h = gncx_ram_alloc_colored(src.size(), 1, 2, 3);
    uint8_t* p = gncx_ram_get_ptr(h);
    gncx_ram_copy_chunk(h, 0, src.data(), 0, src.size());
    CHECK(std::memcmp(p, src.data(), src.size()) == 0);
    gncx_ram_copy_chunk(h, src.size() - 10, src.data(), 5, 10);
    CHECK(p[src.size() - 10] == 5 && p[src.size() - 1] == 14);
    gncx_ram_copy_chunk(h, 0, src.data(), 0, 0);
    gncx_ram_free(h);
    for (void* b : hs) gncx_ram_free(b);
    gncx_ram_free(nullptr);
    CHECK(gncx_ram_get_ptr(nullptr) == nullptr);
}

static void layer_coordinate() {
    for (int32_t total = 1; total <= 80; total += 7)
        for (int32_t layer = -2; layer < total + 2; ++layer)
            for (int32_t k = -1; k < 20; k += 4) {
                int32_t rel = 0, dist = 0, crivo = 0, hemi = 0;
                gncx_genome_get_layer_coordinate(layer, total, k, &rel, &dist, &crivo, &hemi);
            }
}

static void slot_manager() {
    const uint32_t frames[] = {1, 63, 64, 65, 300, 512, 100000};
    for (uint32_t mf : frames) {
        void* g = gncx_geo_mm_create(mf);
        CHECK(g);
        std::vector<std::vector<uint32_t>> live;
        uint8_t k, d, r;
        uint32_t idx;
        for (int i = 0; i < 600; ++i) {
            const uint8_t hint = static_cast<uint8_t>((i * 37) & 0xff);
            if (gncx_geo_alloc(g, hint, &k, &d, &r, &idx) != 0) live.push_back({k, d, r, idx});
            if (i % 5 == 4 && !live.empty()) {
                const auto s = live[live.size() / 2];
                gncx_geo_free(g, static_cast<uint8_t>(s[0]), static_cast<uint8_t>(s[1]), static_cast<uint8_t>(s[2]),
                              s[3]);
                live.erase(live.begin() + static_cast<long>(live.size() / 2));
            }
        }
        // frees of values that were never handed out
        gncx_geo_free(g, 255, 255, 255, 0xffffffffu);
        gncx_geo_free(g, 0, 9, 9, 1u << 30);
        CHECK(gncx_geo_used(g) <= gncx_geo_capacity(g));
        (void)gncx_geo_fragmentation(g);
        gncx_geo_mm_destroy(g);
    }
    gncx_geo_mm_destroy(nullptr);
    CHECK(gncx_geo_used(nullptr) == 0 && gncx_geo_capacity(nullptr) == 0);
}

static void no_device_paths() {
    // every compute entry point reports the missing device and leaves its outputs alone
    std::vector<uint8_t> w(144 * 16, 1);
    std::vector<float> x(4096, 1.0f), y(4096, 7.0f);
    gncx_xfold_universal_matvec(w.data(), 0, GNCX_Q4_K, x.data(), nullptr, 256, 16, y.data(), nullptr);
    CHECK(gncx_hip_last_status() != 0 && y[0] == 7.0f);
    GNCXTelemetryStats t{};
    gncx_xfold_universal_matbatch(w.data(), 0, GNCX_Q4_K, x.data(), 2, 256, 8, y.data(), &t);
    CHECK(gncx_hip_last_status() != 0 && t.total_macs_equivalent == 2u * 256u * 8u);
    gncx_mqa_attention_step_ext(x.data(), x.data(), x.data(), y.data(), y.data(), 3, 4, 2, 64, 0.125f, 0, 1, x.data());
    CHECK(gncx_hip_last_status() != 0);
    gncx_hip_weight_forget(nullptr);
    gncx_hip_kv_forget(nullptr);
    CHECK(gncx_hip_set_host_coherence(2) == 0);
    gncx_hip_host_flush(nullptr);
    gncx_lora_init_adapter(x.data(), y.data(), 4, 4, 2, 1);
    CHECK(gncx_hip_last_status() != 0);
    CHECK(std::strlen(gncx_hip_last_error()) >= 0);
}

int main(int argc, char** argv) {
    const char* dir = argc > 1 ? argv[1] : "/tmp";
    file_mapping(dir);
    host_buffers();
    layer_coordinate();
    slot_manager();
    no_device_paths();
    std::printf("host exports clean under the sanitizers\n");
    return 0;
}

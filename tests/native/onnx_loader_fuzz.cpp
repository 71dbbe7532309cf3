// Host-only build of the ONNX decoder (onnx_amd/csrc/lx_onnx.cpp) under AddressSanitizer and
// UndefinedBehaviorSanitizer, driven by seeded mutations of well-formed models: truncation, bit
// flips, runs of 0xFF bytes and inserted random bytes.  Every load must either succeed or return
// one of the decoder's own statuses; the sanitizers turn any read outside the buffer, use after
// free, leak or undefined arithmetic into a non-zero exit.
//
// The decoder's few calls into the rest of the library are defined below for a process with no
// device: the library reports itself uninitialised, so no initializer is uploaded and no device
// storage, capture or event exists to release.
//
// usage: onnx_loader_fuzz SEED N MODEL...
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "../../include/lonnx.h"
#include "../../onnx_amd/csrc/lx_graph.h"
#include "../../onnx_amd/csrc/lx_internal.h"

namespace lx {
static std::string g_error;
int api_set_error(int code, const std::string &message) {
    g_error = message;
    return code;
}
bool api_initialized() { return false; }
// element sizes of the types the library stores (Float16 and BFloat16 have none)
int64_t api_esize(int dt) {
    switch (dt) {
    case LX_BOOL: case LX_INT8: case LX_UINT8: return 1;
    case LX_INT16: case LX_UINT16: return 2;
    case LX_INT32: case LX_UINT32: case LX_FLOAT: return 4;
    case LX_INT64: case LX_UINT64: case LX_DOUBLE: return 8;
    default: return 0;
    }
}
Storage::~Storage() {}
GraphCapture::~GraphCapture() {}
EventPool::~EventPool() {}
}  // namespace lx

extern "C" int lx_tensor_alloc(int32_t, int32_t, const int64_t *, lx_tensor *) { return LX_ERR_NOT_INITIALIZED; }
extern "C" int lx_tensor_upload(lx_tensor *, const void *, int64_t) { return LX_ERR_NOT_INITIALIZED; }
extern "C" int lx_tensor_free(lx_tensor *) { return LX_OK; }

static std::vector<unsigned char> read_file(const char *path) {
    std::vector<unsigned char> b;
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "cannot open %s\n", path); exit(2); }
    int c;
    while ((c = fgetc(f)) != EOF) b.push_back((unsigned char)c);
    fclose(f);
    return b;
}

int main(int argc, char **argv) {
    if (argc < 4) { fprintf(stderr, "usage: %s SEED N MODEL...\n", argv[0]); return 2; }
    std::mt19937_64 rng(strtoull(argv[1], nullptr, 10));
    const int n = atoi(argv[2]);
    std::vector<std::vector<unsigned char>> seeds;
    for (int i = 3; i < argc; i++) seeds.push_back(read_file(argv[i]));
    int loaded = 0, refused = 0;
    for (int it = 0; it < n; it++) {
        std::vector<unsigned char> b = seeds[it % seeds.size()];
        switch ((it / seeds.size()) % 4) {
        case 0: b.resize(rng() % (b.size() + 1)); break;
        case 1:
            for (int k = 1 + rng() % 8; k > 0; k--) b[rng() % b.size()] ^= (unsigned char)(1u << (rng() % 8));
            break;
        case 2: {
            const size_t p = rng() % b.size();
            for (size_t k = 1 + rng() % 9, j = 0; j < k && p + j < b.size(); j++) b[p + j] = 0xff;
            break;
        }
        default: {
            const size_t p = rng() % b.size();
            std::vector<unsigned char> ins(1 + rng() % 15);
            for (auto &x : ins) x = (unsigned char)rng();
            b.insert(b.begin() + p, ins.begin(), ins.end());
        }
        }
        lx_graph *g = nullptr;
        const int st = lx_graph_load_onnx(b.data(), (int64_t)b.size(), &g);
        if (st == LX_OK) {
            loaded++;
            delete g;
        } else if ((st == LX_ERR_INVALID_ARGUMENT || st == LX_ERR_NOT_SUPPORTED) && !g && !lx::g_error.empty()) {
            refused++;
        } else {
            fprintf(stderr, "mutation %d: status %d, graph %p, message '%s'\n", it, st, (void *)g, lx::g_error.c_str());
            return 1;
        }
        lx::g_error.clear();
    }
    printf("loaded %d refused %d\n", loaded, refused);
    return 0;
}

// ckpt_fuzz.cpp -- test driver: the checkpoint reader's host code (moa_ckpt.hip) built with
// AddressSanitizer and UndefinedBehaviorSanitizer, run over a directory of safetensors files
// (well-formed ones and mutations: truncations, flipped bytes, bad lengths and offsets, deep
// nesting, escapes). For every file it opens, it reads every tensor's description and bytes and
// asks for the global scale of every F32 tensor; files it rejects must be rejected cleanly. Any
// sanitizer report aborts the run with a non-zero status. No device is touched.
#include <dirent.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../include/moa_ckpt.h"

// The library's error recorder (moa_api.hip in the full build).
namespace moa {
static std::string g_last;
int set_error(int code, const char* msg) {
    g_last = msg;
    return code;
}
}  // namespace moa

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s <dir>\n", argv[0]);
        return 2;
    }
    DIR* d = opendir(argv[1]);
    if (!d) return 2;
    std::vector<std::string> files;
    while (dirent* e = readdir(d))
        if (e->d_name[0] != '.') files.push_back(std::string(argv[1]) + "/" + e->d_name);
    closedir(d);
    int opened = 0, rejected = 0, tensors = 0;
    for (const std::string& f : files) {
        moa_ckpt* c = nullptr;
        const int rc = moa_ckpt_open(f.c_str(), &c);
        if (rc != MOA_SUCCESS) {
            if (rc != MOA_ERROR_FORMAT && rc != MOA_ERROR_IO) {
                std::fprintf(stderr, "%s: unexpected code %d (%s)\n", f.c_str(), rc, moa::g_last.c_str());
                return 1;
            }
            if (c) return 1;  // a rejected open hands back no handle
            ++rejected;
            continue;
        }
        ++opened;
        int n = 0;
        moa_ckpt_count(c, &n);
        for (int i = 0; i < n; ++i) {
            const char* name = nullptr;
            if (moa_ckpt_name(c, i, &name) != MOA_SUCCESS) return 1;
            const char* dtype = nullptr;
            int64_t shape[8];
            int ndim = 0;
            uint64_t nbytes = 0;
            if (moa_ckpt_info(c, name, &dtype, shape, &ndim, &nbytes) != MOA_SUCCESS) return 1;
            std::vector<unsigned char> buf(nbytes ? nbytes : 1);
            if (moa_ckpt_read(c, name, buf.data(), nbytes) != MOA_SUCCESS) return 1;
            if (nbytes && moa_ckpt_read(c, name, buf.data(), nbytes - 1) == MOA_SUCCESS) return 1;
            float g = 0.0f;
            (void)moa_ckpt_global_scale(c, name, &g);
            ++tensors;
        }
        if (moa_ckpt_info(c, "no such tensor", nullptr, nullptr, nullptr, nullptr) != MOA_ERROR_NOT_FOUND &&
            moa_ckpt_info(c, "no such tensor", nullptr, nullptr, nullptr, nullptr) != MOA_ERROR_INVALID_VALUE)
            return 1;
        moa_ckpt_close(c);
    }
    std::printf("files %zu opened %d rejected %d tensors %d\n", files.size(), opened, rejected, tensors);
    return 0;
}

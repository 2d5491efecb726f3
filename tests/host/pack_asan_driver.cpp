// Host-only AddressSanitizer driver for the GGUF parser (pack.cpp): open
// each pack given on the command line, describe it, read every tensor and a
// few metadata keys, close it.  Built and run by run_pack_asan.sh; no GPU.
#include "pxs.h"
#include <cstdio>
#include <string>
#include <vector>
#include <cstdlib>
int main(int argc, char ** argv) {
    int ok = 0, bad = 0;
    for (int i = 1; i < argc; ++i) {
        pxs_pack * p = nullptr;
        if (pxs_pack_open(argv[i], &p) != 0) { ++bad; continue; }
        ++ok;
        size_t n = pxs_pack_describe(p, nullptr, 0);
        std::string buf(n, '\0');
        pxs_pack_describe(p, &buf[0], n);
        // read every tensor named in the description
        size_t pos = 0;
        while ((pos = buf.find("{\"name\":\"", pos)) != std::string::npos) {
            pos += 9;
            size_t end = buf.find("\",\"n_dims\"", pos);
            std::string name = buf.substr(pos, end - pos);
            size_t nb = 0;
            pxs_pack_read_tensor(p, name.c_str(), nullptr, 0, &nb);
            std::vector<unsigned char> data(nb + 1);
            pxs_pack_read_tensor(p, name.c_str(), data.data(), nb, &nb);
            uint32_t v; float f; int b; char s[64];
            pxs_pack_metadata_u32(p, "general.alignment", 0, &v);
            pxs_pack_metadata_f32(p, "pixal3d.texture_decoder.norm_eps", 0, &f);
            pxs_pack_metadata_bool(p, "pixal3d.shape_flow_1024.share_mod", 0, &b);
            pxs_pack_metadata_string(p, "general.name", 0, s, sizeof(s));
        }
        pxs_pack_close(p);
    }
    std::printf("opened %d rejected %d\n", ok, bad);
    return 0;
}

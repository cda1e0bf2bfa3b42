// Host-only driver of the model-file parser (safetensors.cpp) and the graph search
// (model_graph.cpp), for sanitizer builds (`make asan`): parses every file named on the
// command line as ppocr_rh_create_from_safetensors, ppocr_model_find_rec_head and
// ppocr_rn_create_from_model do, and prints how many were accepted and refused (with
// --neck first, also the neck each accepted file holds).  A crash, an AddressSanitizer report or an
// UndefinedBehaviorSanitizer finding ends the process with a non-zero status.
#include <cstdio>
#include <string>

#include "model_graph.hpp"

namespace ppocr {
// The library's error channel (api.hip) is not linked here: the last message is kept.
static std::string g_msg;
int fail(int code, const std::string& msg) {
    g_msg = msg;
    return code;
}
}  // namespace ppocr

int main(int argc, char** argv) {
    int accepted = 0, refused = 0, necks = 0;
    bool show = false;
    for (int i = 1; i < argc; ++i) {
        if (std::string(argv[i]) == "--neck") {
            show = true;
            continue;
        }
        ppocr::StFile f;
        int rc = f.open(argv[i]);
        if (rc == 0) {
            // every tensor's bytes are touched, as the head upload reads them
            unsigned sum = 0;
            for (const char* name : {"linear_8.w_0", "linear_8.b_0"})
                if (const ppocr::StTensor* t = f.find(name))
                    for (size_t b = 0; b < t->bytes; b += 997) sum += t->data[b];
            (void)sum;
            ppocr::RecHeadNames r;
            rc = ppocr::find_rec_head(f, &r);
            ppocr::RecNeckNames nk;
            const int nrc = rc == 0 ? ppocr::find_rec_neck(f, &nk) : rc;
            if (show && nrc != 0) std::printf("%s: %s\n", argv[i], ppocr::g_msg.c_str());
            if (nrc == 0) {
                ++necks;
                if (show) {
                    std::printf("neck dim %lld heads %lld hidden %lld scale %.9g blocks %zu lnf %s %s eps %g input %s shortcut %s\n",
                                (long long)nk.dim, (long long)nk.heads, (long long)nk.hidden, nk.scale,
                                nk.blocks.size(), nk.lnf_w.c_str(), nk.lnf_b.c_str(), nk.lnf_eps, nk.input.c_str(),
                                nk.shortcut.c_str());
                    for (const auto& b : nk.blocks)
                        std::printf("  block ln1 %s %s %g qkv %s %s proj %s %s ln2 %s %s %g fc1 %s %s fc2 %s %s\n",
                                    b.ln1_w.c_str(), b.ln1_b.c_str(), b.ln1_eps, b.qkv_w.c_str(), b.qkv_b.c_str(),
                                    b.proj_w.c_str(), b.proj_b.c_str(), b.ln2_w.c_str(), b.ln2_b.c_str(), b.ln2_eps,
                                    b.fc1_w.c_str(), b.fc1_b.c_str(), b.fc2_w.c_str(), b.fc2_b.c_str());
                }
            }
        }
        (rc == 0 ? accepted : refused)++;
    }
    std::printf("accepted %d refused %d necks %d\n", accepted, refused, necks);
    return 0;
}

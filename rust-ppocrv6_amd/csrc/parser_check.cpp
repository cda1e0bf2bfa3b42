// Host-only driver of the model-file parser (safetensors.cpp) and the graph search
// (model_graph.cpp), for sanitizer builds (`make asan`): parses every file named on the
// command line as ppocr_rh_create_from_safetensors and ppocr_model_find_rec_head do, and
// prints how many were accepted and refused.  A crash, an AddressSanitizer report or an
// UndefinedBehaviorSanitizer finding ends the process with a non-zero status.
#include <cstdio>
#include <string>

#include "model_graph.hpp"

namespace ppocr {
// The library's error channel (api.hip) is not linked here: only the status matters.
int fail(int code, const std::string&) { return code; }
}  // namespace ppocr

int main(int argc, char** argv) {
    int accepted = 0, refused = 0;
    for (int i = 1; i < argc; ++i) {
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
        }
        (rc == 0 ? accepted : refused)++;
    }
    std::printf("accepted %d refused %d\n", accepted, refused);
    return 0;
}

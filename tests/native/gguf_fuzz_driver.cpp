// gguf_fuzz_driver.cpp -- runs both GGUF parsers over files named on the
// command line and prints, per file, one line:
//   <runtime status> <oracle status> <runtime text> | <oracle text>
// for GgufFile::parse (level 0) and parse + Config / QuantizedWeights
// (level 1).  Built under AddressSanitizer / UBSan by
// tests/test_gguf_fuzz.py, so an out-of-bounds read, an overflow or an
// oversized allocation in either parser ends the run with a report.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../oracle/vtq_oracle_e2e.h"
#include "../../vitni-tensor_amd/csrc/vtq_gguf.h"

int main(int argc, char** argv) {
    for (int a = 1; a < argc; a++) {
        FILE* f = std::fopen(argv[a], "rb");
        if (!f) return 2;
        std::vector<uint8_t> buf;
        uint8_t tmp[65536];
        size_t n;
        while ((n = std::fread(tmp, 1, sizeof tmp, f)) > 0) buf.insert(buf.end(), tmp, tmp + n);
        std::fclose(f);
        // an exact-size heap copy: a read one byte past the end is reported
        uint8_t* blob = buf.empty() ? nullptr : static_cast<uint8_t*>(std::malloc(buf.size()));
        if (blob) std::copy(buf.begin(), buf.end(), blob);
        for (int level = 0; level < 2; level++) {
            vtq::gguf::File file;
            vtq::gguf::Model model;
            const char* rmsg = "";
            int rrc = vtq::gguf::parse(blob, buf.size(), &file, &rmsg);
            if (!rrc && level == 1) rrc = vtq::gguf::describe(file, &model, &rmsg);
            const char* omsg = "";
            const int orc = vtqo_gguf_parse(blob, buf.size(), level, &omsg);
            std::printf("%d %d %s | %s\n", rrc, orc, rmsg, omsg);
        }
        std::free(blob);
    }
    return 0;
}

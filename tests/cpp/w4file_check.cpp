// w4file_check.cpp -- runs the prepacked-W4 file reader (longhornai_amd/
// csrc/w4file.cpp) on each file named on the command line and prints one
// line per file: "<status> <path> <message>".  Built with AddressSanitizer
// and UndefinedBehaviorSanitizer (tests/cpp/Makefile, bin/w4file_asan), so a
// read outside a buffer, an overflow or a leak in the parser ends the run
// with a sanitizer report instead of passing silently.
#include <cstdio>
#include <string>

#include "w4file.hpp"

int main(int argc, char** argv) {
    for (int i = 1; i < argc; ++i) {
        lhq::W4File f;
        std::string err;
        const int st = lhq::w4file_read("w4file_check", argv[i], f, err);
        std::printf("%d %s %s\n", st, argv[i], st ? err.c_str() : "ok");
    }
    return 0;
}

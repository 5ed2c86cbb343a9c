// Entry point of the C++ suites (GoogleTest's gtest_main equivalent).
#include <gtest/gtest.h>

int main(int argc, char** argv) {
    testing::InitGoogleTest(&argc, argv);
    return RUN_ALL_TESTS();
}

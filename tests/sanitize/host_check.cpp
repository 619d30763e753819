// Runs libgtmoe's host-side C++ under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by tests/sanitize/Makefile):
//  * gtmoe_encode_rows (Rows.Append, lowprecision/rows.go:38-79) on seeded
//    rows of many widths at every precision, bit for bit against the
//    oracle's encoder;
//  * the weights-file reader (ReadBinaryKeepingCompressed,
//    weightfile/binaryfile.go:157-372) on every file named on the command
//    line: every entry read back, then every cut of the file (each prefix)
//    and corrupted copies (bytes set to 0x00, 0xff or flipped) opened and,
//    when accepted, read in full.
// Exits 0 when every check held and no sanitizer fired (the sanitizers
// abort on their first report).
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <random>
#include <string>
#include <vector>

#include "gtmoe.h"

extern "C" void gtmoe_oracle_encode_rows(int precision, int rows, int width, const double *values, float *f32_out,
                                         int8_t *i8_out, uint8_t *fp4_out, float *scales_out);

static int failures = 0;

#define CHECK(cond, ...)                          \
    do {                                          \
        if (!(cond)) {                            \
            fprintf(stderr, "FAILED: " __VA_ARGS__); \
            fprintf(stderr, "\n");                \
            ++failures;                           \
        }                                         \
    } while (0)

static void check_encoder()
{
    std::mt19937_64 gen(7);
    std::normal_distribution<double> normal(0.0, 0.02);
    const int widths[] = {1, 2, 15, 16, 17, 31, 33, 64, 100, 257};
    for (int precision : {GTMOE_FLOAT32, GTMOE_INT8, GTMOE_FP4}) {
        for (int width : widths) {
            const int rows = 5;
            std::vector<double> v((size_t)rows * width);
            for (double &x : v) x = normal(gen);
            v[0] = 0.0;
            if (width > 3) v[3] = -v[2];  // a tie in magnitude
            const int blocks = (width + 15) / 16;
            const size_t code_bytes = precision == GTMOE_FLOAT32 ? (size_t)rows * width * 4
                                      : precision == GTMOE_INT8  ? (size_t)rows * width
                                                                 : (size_t)rows * ((width + 1) / 2);
            std::vector<uint8_t> got(code_bytes), want(code_bytes);
            std::vector<float> gs((size_t)rows * blocks), ws((size_t)rows * blocks);
            const bool scaled = precision != GTMOE_FLOAT32;
            CHECK(gtmoe_encode_rows(precision, rows, width, v.data(), got.data(), scaled ? gs.data() : nullptr) ==
                      GTMOE_OK,
                  "encode precision %d width %d", precision, width);
            gtmoe_oracle_encode_rows(precision, rows, width, v.data(), (float *)want.data(), (int8_t *)want.data(),
                                     want.data(), ws.data());
            CHECK(got == want, "codes differ from the oracle at precision %d width %d", precision, width);
            if (scaled) CHECK(gs == ws, "scales differ from the oracle at precision %d width %d", precision, width);
        }
    }
    CHECK(gtmoe_encode_rows(9, 1, 4, nullptr, nullptr, nullptr) == GTMOE_ERR_INVALID_ARGUMENT, "bad precision");
    CHECK(gtmoe_encode_rows(GTMOE_INT8, 1, 0, nullptr, nullptr, nullptr) == GTMOE_ERR_INVALID_ARGUMENT, "width 0");
}

// Open `path` and read every entry in full; returns whether the file opened.
// `intact`: the file is one the writer made, so every name must be found
// again (a corrupted name may hold a NUL byte, which a C string cuts).
static bool read_all(const char *path, bool intact = false)
{
    gtmoe_weights_file *f = nullptr;
    char err[512];
    if (gtmoe_weights_file_open(path, &f, err, (int32_t)sizeof err) != GTMOE_OK) {
        CHECK(f == nullptr, "a refused file left a handle");
        CHECK(strlen(err) > 0, "a refused file gave no message");
        return false;
    }
    int32_t n = 0;
    CHECK(gtmoe_weights_file_count(f, &n) == GTMOE_OK, "count");
    for (int32_t i = 0; i < n; ++i) {
        char name[256];
        int32_t stored = 0, precision = 0, found = -2;
        int64_t rows = 0, width = 0, count = 0;
        CHECK(gtmoe_weights_file_entry(f, i, name, (int32_t)sizeof name, &stored, &precision, &rows, &width, &count) ==
                  GTMOE_OK,
              "entry %d", i);
        CHECK(gtmoe_weights_file_find(f, name, &found) == GTMOE_OK, "find %s", name);
        if (intact) CHECK(found == i, "find %s gave %d, not %d", name, found, i);
        if (stored != GTMOE_STORED_ROWS) {
            std::vector<double> v((size_t)count);
            (void)gtmoe_weights_file_values(f, i, v.data(), count);
            (void)gtmoe_weights_file_rows(f, i, nullptr, 0, nullptr, 0);  // refused: plain values
        } else {
            const int64_t blocks = (width + 15) / 16;
            const int64_t bytes = precision == GTMOE_FLOAT64   ? rows * width * 8
                                  : precision == GTMOE_FLOAT32 ? rows * width * 4
                                  : precision == GTMOE_INT8    ? rows * width
                                                               : rows * ((width + 1) / 2);
            const int64_t scales = (precision == GTMOE_INT8 || precision == GTMOE_FP4) ? rows * blocks : 0;
            std::vector<uint8_t> codes((size_t)bytes + 1);
            std::vector<float> sc((size_t)scales + 1);
            // an unbalanced split of codes and scales is refused here, not read past
            (void)gtmoe_weights_file_rows(f, i, codes.data(), bytes, sc.data(), scales);
            std::vector<double> v(1);
            (void)gtmoe_weights_file_values(f, i, v.data(), 1);  // refused: compressed rows
        }
        (void)gtmoe_weights_file_entry(f, n, nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr);
    }
    (void)gtmoe_weights_file_error(f);
    gtmoe_weights_file_close(f);
    return true;
}

static std::vector<uint8_t> slurp(const char *path)
{
    std::vector<uint8_t> b;
    FILE *fp = fopen(path, "rb");
    if (!fp) return b;
    uint8_t buf[4096];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, fp)) > 0) b.insert(b.end(), buf, buf + n);
    fclose(fp);
    return b;
}

static void spill(const std::string &path, const uint8_t *data, size_t n)
{
    FILE *fp = fopen(path.c_str(), "wb");
    if (n) fwrite(data, 1, n, fp);
    fclose(fp);
}

static void check_file(const char *path, const std::string &scratch)
{
    CHECK(read_all(path, true), "the intact file %s was refused", path);
    const std::vector<uint8_t> bytes = slurp(path);
    // every cut: a file cut short is refused (the last cut is the file itself)
    int accepted = 0;
    for (size_t cut = 0; cut < bytes.size(); ++cut) {
        spill(scratch, bytes.data(), cut);
        accepted += read_all(scratch.c_str());
    }
    CHECK(accepted == 0, "%d cuts of %s were accepted", accepted, path);
    // corrupted copies: every byte position at a stride, three ways
    const size_t stride = bytes.size() > 4096 ? bytes.size() / 2048 : 1;
    std::vector<uint8_t> bad = bytes;
    for (size_t pos = 0; pos < bytes.size(); pos += stride) {
        for (int how = 0; how < 3; ++how) {
            bad[pos] = how == 0 ? 0x00 : how == 1 ? 0xff : (uint8_t)(bytes[pos] ^ 0x5a);
            spill(scratch, bad.data(), bad.size());
            (void)read_all(scratch.c_str());
        }
        bad[pos] = bytes[pos];
    }
}

int main(int argc, char **argv)
{
    check_encoder();
    const std::string scratch = std::string(getenv("TMPDIR") ? getenv("TMPDIR") : "/tmp") + "/gtmoe_san_" +
                                std::to_string((long)getpid());
    for (int i = 1; i < argc; ++i) check_file(argv[i], scratch);
    unlink(scratch.c_str());
    CHECK(!read_all("/nonexistent/gtmoe.weights"), "a missing file opened");
    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("host_check: encoder and %d weights file(s) clean\n", argc - 1);
    return 0;
}

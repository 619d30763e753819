// Host-side reads from an opened GoTransformers binary weights file, shared
// by the file entry points and the layer load.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

#include "gtmoe.h"

namespace gtmoe {

enum StoredAs { kStoredFloat64 = 1, kStoredFloat32 = 2, kStoredBFloat16 = 3, kStoredRows = 4 };

struct FileEntryInfo {
    int stored_as = 0;
    int precision = -1;  // compressed rows only
    uint64_t rows = 0, width = 0;
    uint64_t count = 0;  // plain values, or rows * width
    // compressed rows: bytes of the list the precision reads and scales
    uint64_t code_bytes = 0, scale_count = 0;
};

// index of `name`, or -1
int file_find(const gtmoe_weights_file *f, const std::string &name);
FileEntryInfo file_info(const gtmoe_weights_file *f, int index);
// a plain parameter as float64; error text in `err`
int32_t file_values(gtmoe_weights_file *f, int index, std::vector<double> &out, std::string &err);
// a compressed parameter: codes as stored (float64, float32, int8 or packed
// FP4 bytes) and its float32 scales
int32_t file_rows(gtmoe_weights_file *f, int index, std::vector<uint8_t> &codes, std::vector<float> &scales,
                  std::string &err);

}  // namespace gtmoe

// GoTransformers binary weights files (weightfile/binaryfile.go): the index
// of a file, its values on the host, and a mixture-of-experts layer's
// parameters moved from the file into the layer's device buffers without a
// float64 copy of the compressed rows.
//
// Format (little endian), as written by writeVersionOne / writeVersionTwo
// (binaryfile.go:63-138):
//   "GOTRANSFORMERS-WEIGHTS-1" u32 n, then per parameter: u32 name length,
//       name, u64 count, count float64
//   "GOTRANSFORMERS-WEIGHTS-2" u32 n, then per parameter: u32 name length,
//       name, u8 stored-as, then
//       1 (float64)  u64 count, count float64
//       2 (float32)  u64 count, count float32
//       3 (bfloat16) u64 count, count uint16 (the upper half of a float32)
//       4 (compressed rows) u8 precision, u64 rows, u64 width, then five
//         lists, each u64 count + values: float64 values, float32 values,
//         int8 values, FP4 bytes, float32 scales
// The checks follow ReadBinaryKeepingCompressed (binaryfile.go:156-372):
// a count may not exceed what the rest of the file could hold, names are
// unique, unknown storage kinds and precisions are errors, and the value and
// scale bytes of compressed rows together must be what their shape needs
// (rows.go:172-203).  The layer upload then checks each array on its own.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "gtmoe.h"
#include "weightfile.h"

using namespace gtmoe;

namespace {

const char kMarker1[] = "GOTRANSFORMERS-WEIGHTS-1";
const char kMarker2[] = "GOTRANSFORMERS-WEIGHTS-2";
constexpr size_t kMarkerLength = 24;

struct List {
    uint64_t count = 0;
    uint64_t offset = 0;  // file offset of the first value
};

struct Entry {
    std::string name;
    int stored_as = 0;
    List values;  // plain parameters
    // compressed rows
    int precision = -1;
    uint64_t rows = 0, width = 0;
    List f64, f32, i8, fp4, scales;
};

}  // namespace

struct gtmoe_weights_file {
    FILE *fp = nullptr;
    uint64_t size = 0;
    int version = 0;
    std::vector<Entry> entries;
    std::unordered_map<std::string, int> by_name;
    std::string error;
};

namespace {

struct Reader {
    FILE *fp;
    uint64_t size;
    uint64_t pos = 0;
    bool read(void *dst, size_t n)
    {
        if (n == 0) return true;
        if (pos + n > size || fread(dst, 1, n, fp) != n) return false;
        pos += n;
        return true;
    }
    bool skip(uint64_t n)
    {
        if (pos + n > size) return false;
        if (n && fseeko(fp, (off_t)n, SEEK_CUR) != 0) return false;
        pos += n;
        return true;
    }
};

int32_t file_fail(gtmoe_weights_file *f, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    f->error = buf;
    return GTMOE_ERR_INVALID_ARGUMENT;
}

// u64 count of a list of `bytes_per_value`-byte values, then skip them
int32_t read_list(gtmoe_weights_file *f, Reader &r, const std::string &name, const char *what, uint64_t bytes_per_value,
                  List &out)
{
    uint64_t count = 0;
    if (!r.read(&count, 8))
        return file_fail(f, "could not read the %s count of parameter \"%s\"", what, name.c_str());
    if (count > f->size / bytes_per_value)
        return file_fail(f, "parameter \"%s\" says it has %llu %s, which is more than the file can hold", name.c_str(),
                         (unsigned long long)count, what);
    out.count = count;
    out.offset = r.pos;
    if (!r.skip(count * bytes_per_value))
        return file_fail(f, "could not read the %s of parameter \"%s\"", what, name.c_str());
    return GTMOE_OK;
}

uint64_t blocks_of(uint64_t width) { return (width + 15) / 16; }

int32_t parse(gtmoe_weights_file *f)
{
    Reader r{f->fp, f->size};
    char marker[kMarkerLength];
    if (!r.read(marker, kMarkerLength)) return file_fail(f, "this is not a binary weights file");
    if (memcmp(marker, kMarker1, kMarkerLength) == 0) f->version = 1;
    else if (memcmp(marker, kMarker2, kMarkerLength) == 0) f->version = 2;
    else return file_fail(f, "this is not a binary weights file");
    uint32_t n = 0;
    if (!r.read(&n, 4)) return file_fail(f, "could not read how many parameters are saved");
    for (uint32_t i = 0; i < n; ++i) {
        Entry e;
        uint32_t len = 0;
        if (!r.read(&len, 4)) return file_fail(f, "could not read the name length of parameter %u", i);
        if (len > f->size)
            return file_fail(f, "parameter %u says its name is %u bytes long, which is bigger than the file", i, len);
        e.name.resize(len);
        if (!r.read(&e.name[0], len)) return file_fail(f, "could not read the name of parameter %u", i);
        if (f->by_name.count(e.name)) return file_fail(f, "parameter \"%s\" is in the file twice", e.name.c_str());
        int32_t rc = GTMOE_OK;
        if (f->version == 1) {
            e.stored_as = kStoredFloat64;
            rc = read_list(f, r, e.name, "values", 8, e.values);
        } else {
            uint8_t how = 0;
            if (!r.read(&how, 1)) return file_fail(f, "could not read how parameter \"%s\" is stored", e.name.c_str());
            e.stored_as = how;
            switch (how) {
            case kStoredFloat64: rc = read_list(f, r, e.name, "values", 8, e.values); break;
            case kStoredFloat32: rc = read_list(f, r, e.name, "float32 values", 4, e.values); break;
            case kStoredBFloat16: rc = read_list(f, r, e.name, "bfloat16 values", 2, e.values); break;
            case kStoredRows: {
                uint8_t prec = 0;
                if (!r.read(&prec, 1))
                    return file_fail(f, "could not read the precision of compressed parameter \"%s\"", e.name.c_str());
                if (!r.read(&e.rows, 8))
                    return file_fail(f, "could not read the row count of compressed parameter \"%s\"", e.name.c_str());
                if (!r.read(&e.width, 8))
                    return file_fail(f, "could not read the row width of compressed parameter \"%s\"", e.name.c_str());
                const uint64_t most = 2 * f->size;
                if (e.width == 0 || e.width > most || e.rows > most / e.width)
                    return file_fail(f, "compressed parameter \"%s\" says it is %llu rows of %llu values, which does not "
                                        "fit in the file",
                                     e.name.c_str(), (unsigned long long)e.rows, (unsigned long long)e.width);
                e.precision = prec;
                if ((rc = read_list(f, r, e.name, "float64 values", 8, e.f64)) != GTMOE_OK) return rc;
                if ((rc = read_list(f, r, e.name, "float32 values", 4, e.f32)) != GTMOE_OK) return rc;
                if ((rc = read_list(f, r, e.name, "int8 values", 1, e.i8)) != GTMOE_OK) return rc;
                if ((rc = read_list(f, r, e.name, "fp4 values", 1, e.fp4)) != GTMOE_OK) return rc;
                if ((rc = read_list(f, r, e.name, "scales", 4, e.scales)) != GTMOE_OK) return rc;
                // RowsFromSnapshot (rows.go:172-203)
                if (prec > GTMOE_FP4)
                    return file_fail(f, "compressed parameter \"%s\": rows snapshot has an unknown precision %u",
                                     e.name.c_str(), prec);
                const uint64_t blocks = blocks_of(e.width);
                uint64_t have = 0, want = 0;
                switch (prec) {
                case GTMOE_FLOAT64: have = e.f64.count * 8; want = e.rows * e.width * 8; break;
                case GTMOE_FLOAT32: have = e.f32.count * 4; want = e.rows * e.width * 4; break;
                case GTMOE_INT8: have = e.i8.count + e.scales.count * 4; want = e.rows * (e.width + blocks * 4); break;
                default: have = e.fp4.count + e.scales.count * 4; want = e.rows * ((e.width + 1) / 2 + blocks * 4);
                }
                if (have != want)
                    return file_fail(f, "compressed parameter \"%s\": rows snapshot for %llu rows of width %llu has the "
                                        "wrong amount of data",
                                     e.name.c_str(), (unsigned long long)e.rows, (unsigned long long)e.width);
                break;
            }
            default: return file_fail(f, "parameter \"%s\" is stored in an unknown way (%u)", e.name.c_str(), how);
            }
        }
        if (rc != GTMOE_OK) return rc;
        f->by_name[e.name] = (int)f->entries.size();
        f->entries.push_back(std::move(e));
    }
    return GTMOE_OK;
}

bool read_at(gtmoe_weights_file *f, uint64_t offset, void *dst, size_t n)
{
    if (n == 0) return true;
    return fseeko(f->fp, (off_t)offset, SEEK_SET) == 0 && fread(dst, 1, n, f->fp) == n;
}

// A plain parameter's values as float64 (bfloat16 widened through float32,
// binaryfile.go:333-343 and precision.go:73-75).
int32_t read_values(gtmoe_weights_file *f, const Entry &e, std::vector<double> &out)
{
    const uint64_t n = e.values.count;
    out.resize(n);
    bool ok = true;
    if (e.stored_as == kStoredFloat64) {
        ok = read_at(f, e.values.offset, out.data(), n * 8);
    } else if (e.stored_as == kStoredFloat32) {
        std::vector<float> v(n);
        ok = read_at(f, e.values.offset, v.data(), n * 4);
        for (uint64_t i = 0; i < n; ++i) out[i] = v[i];
    } else if (e.stored_as == kStoredBFloat16) {
        std::vector<uint16_t> v(n);
        ok = read_at(f, e.values.offset, v.data(), n * 2);
        for (uint64_t i = 0; i < n; ++i) {
            const uint32_t bits = (uint32_t)v[i] << 16;
            float x;
            memcpy(&x, &bits, 4);
            out[i] = x;
        }
    } else {
        return file_fail(f, "parameter \"%s\" holds compressed rows, not plain values", e.name.c_str());
    }
    return ok ? GTMOE_OK : file_fail(f, "could not read the values of parameter \"%s\"", e.name.c_str());
}

// A compressed parameter's codes (Int8 / FP4 bytes, or the float32 /
// float64 values) and scales.
int32_t read_rows(gtmoe_weights_file *f, const Entry &e, std::vector<uint8_t> &codes, std::vector<float> &scales)
{
    if (e.stored_as != kStoredRows)
        return file_fail(f, "parameter \"%s\" holds plain values, not compressed rows", e.name.c_str());
    const List &v = e.precision == GTMOE_FLOAT64   ? e.f64
                    : e.precision == GTMOE_FLOAT32 ? e.f32
                    : e.precision == GTMOE_INT8    ? e.i8
                                                   : e.fp4;
    const uint64_t bytes = v.count * (e.precision == GTMOE_FLOAT64 ? 8 : e.precision == GTMOE_FLOAT32 ? 4 : 1);
    codes.resize(bytes);
    scales.resize(e.scales.count);
    if (!read_at(f, v.offset, codes.data(), bytes) || !read_at(f, e.scales.offset, scales.data(), e.scales.count * 4))
        return file_fail(f, "could not read the rows of parameter \"%s\"", e.name.c_str());
    return GTMOE_OK;
}

}  // namespace

extern "C" {

int32_t gtmoe_weights_file_open(const char *path, gtmoe_weights_file **out, char *error, int32_t error_capacity)
{
    if (!path || !out) return GTMOE_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    gtmoe_weights_file *f = new gtmoe_weights_file;
    f->fp = fopen(path, "rb");
    int32_t rc = GTMOE_OK;
    if (!f->fp) {
        rc = file_fail(f, "could not open %s", path);
    } else if (fseeko(f->fp, 0, SEEK_END) != 0) {
        rc = file_fail(f, "could not size %s", path);
    } else {
        f->size = (uint64_t)ftello(f->fp);
        rewind(f->fp);
        rc = parse(f);
    }
    if (rc != GTMOE_OK) {
        if (error && error_capacity > 0) snprintf(error, (size_t)error_capacity, "%s: %s", path, f->error.c_str());
        if (f->fp) fclose(f->fp);
        delete f;
        return rc;
    }
    *out = f;
    return GTMOE_OK;
}

int32_t gtmoe_weights_file_close(gtmoe_weights_file *f)
{
    if (!f) return GTMOE_OK;
    if (f->fp) fclose(f->fp);
    delete f;
    return GTMOE_OK;
}

const char *gtmoe_weights_file_error(const gtmoe_weights_file *f) { return f ? f->error.c_str() : ""; }

int32_t gtmoe_weights_file_count(const gtmoe_weights_file *f, int32_t *count)
{
    if (!f || !count) return GTMOE_ERR_INVALID_ARGUMENT;
    *count = (int32_t)f->entries.size();
    return GTMOE_OK;
}

int32_t gtmoe_weights_file_entry(const gtmoe_weights_file *f, int32_t index, char *name, int32_t name_capacity,
                                 int32_t *stored_as, int32_t *precision, int64_t *rows, int64_t *width,
                                 int64_t *count)
{
    if (!f || index < 0 || index >= (int32_t)f->entries.size()) return GTMOE_ERR_INVALID_ARGUMENT;
    const Entry &e = f->entries[(size_t)index];
    if (name && name_capacity > 0) snprintf(name, (size_t)name_capacity, "%s", e.name.c_str());
    if (stored_as) *stored_as = e.stored_as;
    if (precision) *precision = e.precision;
    if (rows) *rows = (int64_t)e.rows;
    if (width) *width = (int64_t)e.width;
    if (count) *count = (int64_t)(e.stored_as == kStoredRows ? e.rows * e.width : e.values.count);
    return GTMOE_OK;
}

int32_t gtmoe_weights_file_find(const gtmoe_weights_file *f, const char *name, int32_t *index)
{
    if (!f || !name || !index) return GTMOE_ERR_INVALID_ARGUMENT;
    auto it = f->by_name.find(name);
    *index = it == f->by_name.end() ? -1 : it->second;
    return GTMOE_OK;
}

int32_t gtmoe_weights_file_values(gtmoe_weights_file *f, int32_t index, double *out, int64_t count)
{
    if (!f || index < 0 || index >= (int32_t)f->entries.size() || (count > 0 && !out)) return GTMOE_ERR_INVALID_ARGUMENT;
    const Entry &e = f->entries[(size_t)index];
    std::vector<double> v;
    int32_t rc = read_values(f, e, v);
    if (rc != GTMOE_OK) return rc;
    if ((int64_t)v.size() != count)
        return file_fail(f, "parameter \"%s\" holds %llu values, not %lld", e.name.c_str(),
                         (unsigned long long)v.size(), (long long)count);
    if (!v.empty()) memcpy(out, v.data(), v.size() * sizeof(double));
    return GTMOE_OK;
}

int32_t gtmoe_weights_file_rows(gtmoe_weights_file *f, int32_t index, void *values, int64_t values_bytes,
                                float *scales, int64_t scale_count)
{
    if (!f || index < 0 || index >= (int32_t)f->entries.size()) return GTMOE_ERR_INVALID_ARGUMENT;
    const Entry &e = f->entries[(size_t)index];
    std::vector<uint8_t> codes;
    std::vector<float> sc;
    int32_t rc = read_rows(f, e, codes, sc);
    if (rc != GTMOE_OK) return rc;
    if ((int64_t)codes.size() != values_bytes || (int64_t)sc.size() != scale_count)
        return file_fail(f, "parameter \"%s\" holds %zu value bytes and %zu scales", e.name.c_str(), codes.size(),
                         sc.size());
    if (!codes.empty()) memcpy(values, codes.data(), codes.size());
    if (!sc.empty()) memcpy(scales, sc.data(), sc.size() * sizeof(float));
    return GTMOE_OK;
}

}  // extern "C"

namespace gtmoe {

int file_find(const gtmoe_weights_file *f, const std::string &name)
{
    auto it = f->by_name.find(name);
    return it == f->by_name.end() ? -1 : it->second;
}

FileEntryInfo file_info(const gtmoe_weights_file *f, int index)
{
    const Entry &e = f->entries[(size_t)index];
    FileEntryInfo i;
    i.stored_as = e.stored_as;
    i.precision = e.precision;
    i.rows = e.rows;
    i.width = e.width;
    i.count = e.stored_as == kStoredRows ? e.rows * e.width : e.values.count;
    if (e.stored_as == kStoredRows) {
        i.code_bytes = e.precision == GTMOE_FLOAT64   ? e.f64.count * 8
                       : e.precision == GTMOE_FLOAT32 ? e.f32.count * 4
                       : e.precision == GTMOE_INT8    ? e.i8.count
                                                      : e.fp4.count;
        i.scale_count = e.scales.count;
    }
    return i;
}

int32_t file_values(gtmoe_weights_file *f, int index, std::vector<double> &out, std::string &err)
{
    const int32_t rc = read_values(f, f->entries[(size_t)index], out);
    if (rc != GTMOE_OK) err = f->error;
    return rc;
}

int32_t file_rows(gtmoe_weights_file *f, int index, std::vector<uint8_t> &codes, std::vector<float> &scales,
                  std::string &err)
{
    const int32_t rc = read_rows(f, f->entries[(size_t)index], codes, scales);
    if (rc != GTMOE_OK) err = f->error;
    return rc;
}

}  // namespace gtmoe

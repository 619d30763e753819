// Host-side quantization: lowprecision.Rows.Append (lowprecision/rows.go:38-79)
// with the encoders of lowprecision/lowprecision.go:56-104, bit-exact.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "gtmoe.h"

namespace {

constexpr int kBlock = 16;  // ValuesPerScale, lowprecision.go:46

// scale = float32(max|v| / largest code magnitude)
float block_scale(const double *v, int n, double largest_code)
{
    double m = 0.0;
    for (int i = 0; i < n; ++i)
        if (fabs(v[i]) > m) m = fabs(v[i]);
    return (float)(m / largest_code);
}

// encodeInt8 (lowprecision.go:66-78): round half away from zero, clamp +-127
int8_t to_int8(double value, double scale)
{
    if (scale == 0) return 0;
    double r = round(value / scale);
    if (r > 127) r = 127;
    if (r < -127) r = -127;
    return (int8_t)r;
}

// encodeFP4 (lowprecision.go:80-96): sign bit 8 for negatives; magnitude
// code = number of halfway points strictly below |v| / scale.
uint8_t to_fp4(double value, double scale)
{
    static const double kHalfway[7] = {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5};
    if (scale == 0) return 0;
    const uint8_t sign = value < 0 ? 8 : 0;
    const double m = fabs(value) / scale;
    uint8_t code = 0;
    while (code < 7 && m > kHalfway[code]) ++code;
    return (uint8_t)(sign | code);
}

}  // namespace

extern "C" int32_t gtmoe_encode_rows(int32_t precision, int32_t rows, int32_t width, const double *values,
                                     void *values_out, float *scales_out)
{
    if (rows < 0 || width <= 0 || (rows > 0 && (!values || !values_out))) return GTMOE_ERR_INVALID_ARGUMENT;
    const int blocks = (width + kBlock - 1) / kBlock;
    if ((precision == GTMOE_INT8 || precision == GTMOE_FP4) && rows > 0 && !scales_out)
        return GTMOE_ERR_INVALID_ARGUMENT;
    for (int r = 0; r < rows; ++r) {
        const double *row = values + (size_t)r * width;
        switch (precision) {
        case GTMOE_FLOAT64:
            memcpy((double *)values_out + (size_t)r * width, row, sizeof(double) * (size_t)width);
            break;
        case GTMOE_FLOAT32: {
            float *out = (float *)values_out + (size_t)r * width;
            for (int i = 0; i < width; ++i) out[i] = (float)row[i];
            break;
        }
        case GTMOE_INT8: {
            int8_t *out = (int8_t *)values_out + (size_t)r * width;
            for (int b = 0; b < blocks; ++b) {
                const int start = b * kBlock, n = start + kBlock < width ? kBlock : width - start;
                const float s = block_scale(row + start, n, 127.0);
                scales_out[(size_t)r * blocks + b] = s;
                for (int i = 0; i < n; ++i) out[start + i] = to_int8(row[start + i], (double)s);
            }
            break;
        }
        case GTMOE_FP4: {
            const int row_bytes = (width + 1) / 2;
            uint8_t *out = (uint8_t *)values_out + (size_t)r * row_bytes;
            memset(out, 0, (size_t)row_bytes);
            for (int b = 0; b < blocks; ++b) {
                const int start = b * kBlock, n = start + kBlock < width ? kBlock : width - start;
                const float s = block_scale(row + start, n, 6.0);
                scales_out[(size_t)r * blocks + b] = s;
                for (int i = start; i < start + n; ++i) {
                    const uint8_t c = to_fp4(row[i], (double)s);
                    out[i / 2] |= (uint8_t)((i % 2) ? (c << 4) : c);
                }
            }
            break;
        }
        default:
            return GTMOE_ERR_INVALID_ARGUMENT;
        }
    }
    return GTMOE_OK;
}

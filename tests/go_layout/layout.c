/* Prints the sizes and field offsets of the C ABI's structs as gcc lays
 * them out, one "struct field offset size" line per field and a "struct
 * sizeof N" line per struct, for tests/test_go_binding.py to compare with
 * the Go mirror types in go/mixtureofexperts/gpu_unix.go. */
#include <stddef.h>
#include <stdio.h>

#include "gtmoe.h"

#define FIELD(s, f) printf(#s " " #f " %zu %zu\n", offsetof(s, f), sizeof(((s *)0)->f))

int main(void)
{
    FIELD(gtmoe_layer_desc, vector_size);
    FIELD(gtmoe_layer_desc, expert_hidden_size);
    FIELD(gtmoe_layer_desc, shared_experts);
    FIELD(gtmoe_layer_desc, routed_experts);
    FIELD(gtmoe_layer_desc, experts_per_token);
    FIELD(gtmoe_layer_desc, precision);
    FIELD(gtmoe_layer_desc, use_hash_routing);
    FIELD(gtmoe_layer_desc, reserved);
    FIELD(gtmoe_layer_desc, clamp_limit);
    printf("gtmoe_layer_desc sizeof %zu\n", sizeof(gtmoe_layer_desc));
    FIELD(gtmoe_rows, precision);
    FIELD(gtmoe_rows, rows);
    FIELD(gtmoe_rows, width);
    FIELD(gtmoe_rows, reserved);
    FIELD(gtmoe_rows, values);
    FIELD(gtmoe_rows, values_bytes);
    FIELD(gtmoe_rows, scales);
    FIELD(gtmoe_rows, scale_count);
    printf("gtmoe_rows sizeof %zu\n", sizeof(gtmoe_rows));
    return 0;
}

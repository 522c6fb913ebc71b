/* SPDX-License-Identifier: MIT
 *
 * K-quant super-block wire formats (GGUF Q4_K / Q6_K) shared by the C99 host
 * code, the oracle and the HIP kernels.
 *
 * The byte layouts are fixed by the GGUF format and therefore match the
 * reference's declarations byte for byte:
 *   block_q4_K  engine/src/third_party/gguf.h:26-32   (144 bytes)
 *   block_q6_K  engine/src/third_party/gguf.h:34-40   (210 bytes)
 *   row sizes   engine/src/third_party/gguf.h:43-53
 *   type codes  engine/src/third_party/gguf.h:15-22
 *
 * Field access in this code base goes through byte offsets (ORN_Q4K_OFF_*,
 * ORN_Q6K_OFF_*) so that device code can read a block from any byte address
 * without relying on host struct packing rules.
 */
#ifndef ORNITH_KQUANT_H
#define ORNITH_KQUANT_H

#include <stdint.h>
#include <stddef.h>

#define ORN_QK_K 256 /* elements per super-block */

typedef enum {
    ORN_TYPE_F32 = 0,
    ORN_TYPE_F16 = 1,
    ORN_TYPE_Q4_0 = 2,
    ORN_TYPE_Q8_0 = 8,
    ORN_TYPE_Q4_K = 12,
    ORN_TYPE_Q6_K = 14
} orn_type;

/* Q4_K: d (fp16) | dmin (fp16) | scales[12] (8 x 6-bit sc, 8 x 6-bit m) | qs[128] */
#define ORN_Q4K_BYTES 144
#define ORN_Q4K_OFF_D 0
#define ORN_Q4K_OFF_DMIN 2
#define ORN_Q4K_OFF_SCALES 4
#define ORN_Q4K_OFF_QS 16

/* Q6_K: ql[128] (low nibbles) | qh[64] (high 2-bit pairs) | scales[16] (int8) | d (fp16) */
#define ORN_Q6K_BYTES 210
#define ORN_Q6K_OFF_QL 0
#define ORN_Q6K_OFF_QH 128
#define ORN_Q6K_OFF_SCALES 192
#define ORN_Q6K_OFF_D 208

typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[ORN_QK_K / 2];
} orn_block_q4k;

typedef struct {
    uint8_t ql[ORN_QK_K / 2];
    uint8_t qh[ORN_QK_K / 4];
    int8_t scales[ORN_QK_K / 16];
    uint16_t d;
} orn_block_q6k;

/* Compile-time layout checks (C99 style: a negative array size fails). */
typedef char orn_q4k_size_check[(sizeof(orn_block_q4k) == ORN_Q4K_BYTES) ? 1 : -1];
typedef char orn_q6k_size_check[(sizeof(orn_block_q6k) == ORN_Q6K_BYTES) ? 1 : -1];

/* Bytes occupied by n_elems elements of a type; 0 for unsupported types.
 * Same contract as ggml_row_size (third_party/gguf.h:43-53). */
static inline size_t orn_row_size(int type, uint64_t n_elems)
{
    switch (type) {
    case ORN_TYPE_F32: return (size_t)(n_elems * 4u);
    case ORN_TYPE_F16: return (size_t)(n_elems * 2u);
    case ORN_TYPE_Q4_0: return (size_t)((n_elems / 32u) * 18u);
    case ORN_TYPE_Q8_0: return (size_t)((n_elems / 32u) * 34u);
    case ORN_TYPE_Q4_K: return (size_t)((n_elems / ORN_QK_K) * ORN_Q4K_BYTES);
    case ORN_TYPE_Q6_K: return (size_t)((n_elems / ORN_QK_K) * ORN_Q6K_BYTES);
    default: return 0;
    }
}

#endif /* ORNITH_KQUANT_H */

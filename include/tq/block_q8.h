/* block_q8.h — the Q8 block: 32 int8 codes sharing one fp32 scale (and the
 * Q4 weight block beside it).
 *
 * Byte layout (36 bytes, no padding): float d at offset 0, int8 q[32] at
 * offset 4.  This is the layout of packer/packer.h:7-11 in the reference, so a
 * block written by the reference's quantize_row_q8 (kernel/quant_x.c:12-33)
 * and one written by this library's kernels are interchangeable byte for byte.
 *
 * When the reference's packer.h has already been included (its include guard
 * PACKER_H is defined) its definition of QK and block_q8 is reused, so both
 * headers can sit in one translation unit.
 */
#ifndef TQ_BLOCK_Q8_H
#define TQ_BLOCK_Q8_H

#include <stdint.h>

#ifndef PACKER_H
#define QK 32
typedef struct {
    float  d;
    int8_t q[QK];
} block_q8;
/* The Q4 weight block (packer/packer.h:9): 32 codes in [-7, 7] stored as
 * code + 8 in nibbles, byte j holding code j in its low nibble and code
 * j + 16 in its high nibble; 20 bytes. */
typedef struct {
    float   d;
    uint8_t q[QK / 2];
} block_q4;
#endif

#ifdef __cplusplus
static_assert(sizeof(block_q8) == 36, "block_q8 must be 36 bytes with no padding");
static_assert(sizeof(block_q4) == 20, "block_q4 must be 20 bytes with no padding");
#else
_Static_assert(sizeof(block_q8) == 36, "block_q8 must be 36 bytes with no padding");
_Static_assert(sizeof(block_q4) == 20, "block_q4 must be 20 bytes with no padding");
#endif

#endif /* TQ_BLOCK_Q8_H */

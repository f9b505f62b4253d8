/*
 * qmm_params.h -- the launch parameter block shared by the host runtime and the gfx950
 * kernels of the small-M affine-quantised matmul.  Plain C layout, passed by value as the
 * single kernel argument.
 */
#ifndef DFQ_QMM_PARAMS_H
#define DFQ_QMM_PARAMS_H

#include <stdint.h>

/* Work decomposition of the fast kernel (a "stream-K" split with a deterministic fix-up):
 *
 *  - output features are cut into T column tiles of 16 (the MFMA N dimension);
 *  - K is cut into nkb k-blocks of kr elements (kr * rows of x must fit in LDS), and each
 *    k-block into SS chunks of CH super-steps (one super-step = the k span that holds
 *    exactly two quantisation groups per lane half, 64..256 elements; a chunk is one
 *    super-step or the 8 groups whose scales one 16-byte load fetches);
 *  - the U = T*SS units (tile, chunk) of one k-block are split into Gkb contiguous ranges
 *    whose sizes differ by at most one (the first U % Gkb get one more), and each
 *    workgroup's range likewise into one range per wave;
 *  - a tile covered by one wave is parked in LDS during the main loop and written to y
 *    after it (the loop itself issues no global stores); a tile shared between waves is
 *    summed in LDS in wave order; a tile shared between workgroups (or k-blocks) is summed
 *    through workspace slots in a fixed order by whichever workgroup arrives last.
 */
typedef struct QmmParams {
    const void* x;          /* [M][K] activations, bf16 or fp16                      */
    const uint32_t* w;      /* [N][K*bits/32] packed codes, element 0 in low bits     */
    const void* scales;     /* [N][K/gs] same dtype as x                              */
    const void* biases;     /* [N][K/gs]                                              */
    const void* lbias;      /* [N] optional linear bias (NULL if none)               */
    void* y;                /* [M][N] output, same dtype as x                         */
    float* slots;           /* workspace: per-tile partial sums                       */
    uint32_t* counters;     /* workspace: per-tile arrival counters (zero at rest)    */
    int32_t M, N, K;
    int32_t T;              /* column tiles of 16                                     */
    int32_t SS;             /* chunks per tile per k-block                            */
    int32_t nkb;            /* k-blocks                                               */
    int32_t Gkb;            /* workgroups per k-block                                 */
    int32_t nslot_kb;       /* partial slots per tile per k-block                     */
    int32_t kr;             /* k elements per k-block                                 */
    int32_t lds_row_stride; /* bytes per staged x row in LDS                          */
    int32_t lds_xsum_off;   /* byte offset of the per-group x sums in LDS             */
    int32_t lds_slot_off;   /* byte offset of the per-wave partial slots in LDS       */
    int32_t lds_ytile_off;  /* byte offset of the per-wave result tiles in LDS        */
    int32_t ytw;            /* result tiles per wave (tiles wholly inside its range)  */
    int32_t wg_base;        /* units per workgroup, rounded down (U / Gkb)            */
    int32_t wg_rem;         /* workgroups with one extra unit (U % Gkb)               */
    uint32_t w_bytes;       /* size of w in bytes (< 2^31)                            */
    uint32_t s_bytes;       /* size of scales (= size of biases) in bytes             */
} QmmParams;

/* Parameters of the generic (stock-op stand-in) kernel. */
typedef struct QmmGenericParams {
    const void* x;
    const uint32_t* w;
    const void* scales;
    const void* biases;
    const void* lbias;
    void* y;
    int32_t M, N, K, bits, gs;
    int32_t xdt, sdt, ydt;  /* 0 bf16, 1 fp16, 2 fp32 */
} QmmGenericParams;

#endif

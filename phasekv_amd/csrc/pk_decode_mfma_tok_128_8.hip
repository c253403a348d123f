// One variant of the MFMA decode kernel for per-token K segments (head_dim 128,
// codes up to 8 bits), in a translation unit of its own so that the variants
// compile in parallel.
#define PK_MFMA_HD 128
#define PK_MFMA_MAXB 8
#define PK_MFMA_TOK 1
#include "pk_decode_mfma.h"

// One variant of the MFMA decode kernel (head_dim 64, codes up to 2 bits, four waves,
// the wave-private group path only), in a translation unit of its own so that the
// variants compile in parallel.
#define PK_MFMA_HD 64
#define PK_MFMA_MAXB 2
#define PK_MFMA_WO 1
#include "pk_decode_mfma.h"

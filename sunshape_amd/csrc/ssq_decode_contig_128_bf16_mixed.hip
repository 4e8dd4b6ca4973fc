// Contiguous-layout decode instantiations: 128-dim bf16 values, passthrough (heavy-block) values.
#include "ssq_decode_contig.h"

SSQ_CONTIG_UNIT(ssq_contig_128_bf16_mixed) { return contig_mixed<8, SSQ_BF16, true>(cp, pl, st); }

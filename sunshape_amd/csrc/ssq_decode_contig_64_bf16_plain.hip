// Contiguous-layout decode instantiations: 64-dim bf16 values, byte codes with or without a mask, 4- and 6-bit packed codes.
#include "ssq_decode_contig.h"

SSQ_CONTIG_UNIT(ssq_contig_64_bf16_plain) { return contig_plain<4, SSQ_BF16, true>(cp, pl, st); }

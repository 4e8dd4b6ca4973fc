// Contiguous-layout decode instantiations: 128-dim bf16 values, byte codes with or without a mask, 4- and 6-bit packed codes.
#include "ssq_decode_contig.h"

SSQ_CONTIG_UNIT(ssq_contig_128_bf16_plain) { return contig_plain<8, SSQ_BF16, true>(cp, pl, st); }

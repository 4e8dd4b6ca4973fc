// Contiguous-layout decode instantiations: 128-dim f16 values, byte codes with or without a mask, 4- and 6-bit packed codes.
#include "ssq_decode_contig.h"

SSQ_CONTIG_UNIT(ssq_contig_128_f16_plain) { return contig_plain<8, SSQ_F16, true>(cp, pl, st); }

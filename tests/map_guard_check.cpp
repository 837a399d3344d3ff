// Host-side check of trmoe::mapped_dest (the destination guard of the mapped
// weight-gradient reduction): reads "off idx stride out_elems" lines from
// stdin and prints one destination per line.  Built by tests/test_grad_maps.py.
#include "trmoe_map.h"

#include <stdio.h>

int main() {
    long long off, idx, stride, lim;
    while (scanf("%lld %lld %lld %lld", &off, &idx, &stride, &lim) == 4)
        printf("%lld\n", (long long)trmoe::mapped_dest(off, idx, stride, lim));
    return 0;
}

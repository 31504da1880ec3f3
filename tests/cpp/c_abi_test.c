/* The C ABI from plain C99: the headers compile as C, and the host-only entry
 * points (no GPU touched) behave as documented.  Built and run by
 * tests/test_c_abi.py; exit status 0 = pass. */
#include <stdio.h>
#include <string.h>

#include "sfa.h"
#include "sfa_layer.h"
#include "sfa_pager.h"

#define CHECK(cond)                                                   \
    do {                                                              \
        if (!(cond)) {                                                \
            fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
            return 1;                                                 \
        }                                                             \
    } while (0)

int main(void) {
    sfa_kv_desc d;
    memset(&d, 0, sizeof d);
    d.n_head = 32;
    d.n_head_kv = 8;
    d.head_dim = 128;
    d.page_size = 256;
    d.kv_type = SFA_KV_F16;
    d.n_pages = 16;
    d.k_pages = d.v_pages = (void *)0x1000; /* never dereferenced by host-only calls */

    CHECK(strcmp(sfa_status_str(SFA_OK), "ok") == 0);
    CHECK(sfa_version() != NULL && sfa_version()[0] != '\0');
    CHECK(sfa_kv_desc_check(&d) == SFA_OK);
    CHECK(sfa_row_bytes(&d) == 256);
    CHECK(sfa_page_bytes(&d) == (size_t)256 * 8 * 256);
    CHECK(sfa_decode_workspace_bytes(&d, 1, 4096) > 0);

    d.head_dim = 96;
    CHECK(sfa_kv_desc_check(&d) == SFA_ERR_UNSUPPORTED);
    d.head_dim = 128;
    d.kv_type = SFA_KV_Q8_0;
    CHECK(sfa_row_bytes(&d) == 136);

    /* host page-table validation: 700 positions need three pages, the third is -1 */
    {
        const int32_t pt[4] = {0, 3, -1, -1};
        const int32_t len_bad[1] = {700};
        const int32_t len_ok[1] = {500};
        CHECK(sfa_page_table_check(&d, pt, 4, len_bad, NULL, 1) == SFA_ERR_INVALID_ARGUMENT);
        CHECK(sfa_page_table_check(&d, pt, 4, len_ok, NULL, 1) == SFA_OK);
    }
    /* the pager rejects a bad configuration without touching the GPU */
    {
        sfa_pager_config c;
        sfa_pager *p = NULL;
        memset(&c, 0, sizeof c);
        c.n_layer = 0;
        CHECK(sfa_pager_create(&c, &p) == SFA_ERR_INVALID_ARGUMENT && p == NULL);
        CHECK(sfa_pager_begin(NULL, NULL, NULL) == SFA_ERR_INVALID_ARGUMENT);
    }
    /* the layer entry points validate before any device work */
    {
        void *p = (void *)0x1000;
        CHECK(sfa_moe_workspace_bytes(3, 2, 512) == (size_t)3 * 2 * 512 * 4);
        CHECK(sfa_mul_mat_vec(p, SFA_KV_F16, (const float *)p, NULL, (float *)p, 1, 100, 64, NULL) ==
              SFA_ERR_UNSUPPORTED);
        CHECK(sfa_rms_norm(NULL, (const float *)p, (float *)p, 1, 256, 1e-5f, NULL) == SFA_ERR_INVALID_ARGUMENT);
        CHECK(sfa_moe_route((const float *)p, 1, 8, 9, (int32_t *)p, (float *)p, NULL) == SFA_ERR_INVALID_ARGUMENT);
    }
    printf("c abi ok\n");
    return 0;
}

/* Embeds the gfx950 code objects built from kernels.hip into libglmssd_hip.so. */
#define BLOB(NAME, FILE)                 \
    .section .rodata.gs_blob_##NAME, "a"; \
    .balign 4096;                        \
    .globl gs_blob_##NAME##_start;       \
    .globl gs_blob_##NAME##_end;         \
gs_blob_##NAME##_start:                  \
    .incbin FILE;                        \
gs_blob_##NAME##_end:                    \
    .byte 0;

BLOB(common, "build/common.hsaco")
BLOB(grouped, "build/grouped.hsaco")
BLOB(gemm, "build/gemm.hsaco")
BLOB(t0, "build/t0.hsaco")
BLOB(t1, "build/t1.hsaco")
BLOB(t8, "build/t8.hsaco")
BLOB(t10, "build/t10.hsaco")
BLOB(t11, "build/t11.hsaco")
BLOB(t12, "build/t12.hsaco")
BLOB(t13, "build/t13.hsaco")
BLOB(t14, "build/t14.hsaco")
BLOB(t16, "build/t16.hsaco")
BLOB(t18, "build/t18.hsaco")
BLOB(t22, "build/t22.hsaco")
BLOB(t23, "build/t23.hsaco")
BLOB(t30, "build/t30.hsaco")

.section .note.GNU-stack,"",@progbits

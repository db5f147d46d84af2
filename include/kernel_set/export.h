/*
 * kernel-set (MI355X build) -- symbol visibility and C linkage helpers.
 *
 * Same macro names as the reference ABI (include/kernel_set/export.h:12-30 of
 * cklxx/kernel-set) so that headers and bindings written against it compile
 * unchanged. This build targets Linux/gfx950 only, so KS_API is always the
 * ELF default-visibility attribute.
 */
#ifndef KERNEL_SET_EXPORT_H_
#define KERNEL_SET_EXPORT_H_

#define KS_API __attribute__((visibility("default")))

#ifdef __cplusplus
#define KS_BEGIN_EXTERN_C extern "C" {
#define KS_END_EXTERN_C }
#else
#define KS_BEGIN_EXTERN_C
#define KS_END_EXTERN_C
#endif

#endif /* KERNEL_SET_EXPORT_H_ */

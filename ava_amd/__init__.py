"""ava_amd: MI355X-native int8 block forward of Ava (see include/ava.h for the C ABI)."""

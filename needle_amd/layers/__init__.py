"""Drop-in layers that route Needle's attention seams to the HIP kernels."""

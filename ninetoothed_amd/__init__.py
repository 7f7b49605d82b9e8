"""ninetoothed_amd: an MI355X-native (gfx950) backend for NineToothed's arrange-and-apply kernels."""

// Package native: the hook through which a build-tagged accelerator replaces
// the CPU forward of EncodeTokens/EmbedBatch.  This file has no build tag and
// no cgo: in the default build accelNew stays nil and nothing changes.
//
// Copy into futon's native/ next to model.go (see INTEGRATION.md for the
// three call sites in model.go and provider.go that consult it).
package native

import "context"

// accelModel runs whole forwards of a validated pack on an accelerator.
// EncodeBatch has EncodeTokensKernel's contract for every sequence
// (model.go:346-457): same validation errors, nil vectors and ctx.Err() on
// cancellation, vectors index-aligned, each equal to its single-sequence
// forward whatever else is in the batch.
type accelModel interface {
	EncodeBatch(ctx context.Context, batch [][]int, outDim int) ([][]float32, error)
	Close() error
}

// accelNew, when set (by an accelerator's build-tagged init), is called by
// newModel after all of its validation, with the same config and tensors.
// A nil model and nil error mean "not available here" (no device): the CPU
// path stays in use.
var accelNew func(cfg *PackConfig, tensors map[string]*Tensor) (accelModel, error)

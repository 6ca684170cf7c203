//go:build !qmoe

// moe_hip_stub.go -- the CPU build (no `qmoe` tag): moeMLP never has a device
// copy, so moeMLP.forward keeps its Go body and decodeLayers its per-token
// loop (moeMLP does not implement batchMixer here).
package model

import "errors"

type qmoeDev struct{}

func (m *moeMLP) uploadQmoe(device int, selectScope int) error {
	return errors.New("built without the qmoe tag")
}

func (m *moeMLP) forwardQmoe(x []float32) []float32 { panic("built without the qmoe tag") }

func (m *moeMLP) closeQmoe() {}

"""Pack declarations of every gfx950 kernel; importing a module registers its specs."""
